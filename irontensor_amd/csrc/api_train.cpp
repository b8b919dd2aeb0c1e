// C ABI entry points for the training step's ops around the contractions: argument validation with
// the reference's error cases (assert! on shapes and precisions becomes IT_ERR_*), library-owned
// scratch for the deterministic reductions, and profiler keys for the step breakdown.
#include <cstdint>
#include <algorithm>
#include <cstring>
#include <string>
#include <vector>

#include "internal.hpp"

using it::fail;

namespace {

std::string i64(int64_t v) { return std::to_string((long long)v); }

bool f32_or_bf16(it_dtype d) { return d == IT_F32 || d == IT_BF16; }

// Times one op under the profiler (no-op otherwise).
struct Prof {
    it_context *ctx;
    std::string key;
    hipEvent_t ev = nullptr;
    Prof(it_context *c, std::string k) : ctx(c) {
        if (ctx->profiling) {
            key = std::move(k);
            it::profile_begin(ctx, key, &ev);
        }
    }
    it_status done(it_status st) {
        if (ctx->profiling) it::profile_end(ctx, key, ev);
        return st;
    }
};

const char *sfx(it_dtype d) { return d == IT_BF16 ? "_bf16" : "_f32"; }

}  // namespace

namespace it {

// (cos, sin) per (position, pair): built once per parameter set on the calling stream, kept in the
// context, and shared by every later call (a graph replay reuses it unchanged).
it_status rope_table(it_context *ctx, int64_t seq, int64_t head_dim, float base, int64_t offset, const void **out) {
    uint32_t base_bits;
    std::memcpy(&base_bits, &base, sizeof base_bits);
    const std::vector<int64_t> key{seq, head_dim, (int64_t)base_bits, offset};
    auto found = ctx->rope_tables.find(key);
    if (found != ctx->rope_tables.end()) {
        *out = found->second;
        return IT_OK;
    }
    if (ctx->capturing)
        return fail(IT_ERR_INVALID, "rope: first use of these parameters during graph capture: "
                                    "run the work once before capturing");
    void *table = nullptr;
    IT_HIP_TRY(hipMalloc(&table, (size_t)(seq * (head_dim / 2)) * 2 * sizeof(float)));
    ctx->rope_tables[key] = table;
    if (const it_status st = launch_rope_table(ctx->stream, seq, head_dim, base, offset, table); st != IT_OK) return st;
    // Ready before any stream uses it (later calls may come from the other stream).
    IT_HIP_TRY(hipStreamSynchronize(ctx->stream));
    *out = table;
    return IT_OK;
}

}  // namespace it

extern "C" {

it_status it_rmsnorm_forward(it_context *ctx, it_dtype dtype_y, int64_t rows, int64_t dim, float eps,
                             const float *x, const float *res, const float *gamma, float *sum_out, void *y) {
    if (!ctx) return fail(IT_ERR_NULL, "rmsnorm: ctx is NULL");
    if (!f32_or_bf16(dtype_y)) return fail(IT_ERR_PRECISION, "rmsnorm: precision mismatch, expected FP32 or BF16");
    if (rows < 0 || dim < 0) return fail(IT_ERR_INVALID, "rmsnorm: negative size");
    if (rows == 0 || dim == 0) return IT_OK;
    if (!x || !gamma || !y) return fail(IT_ERR_NULL, "rmsnorm: NULL buffer");
    Prof p(ctx, std::string("rmsnorm_fwd") + sfx(dtype_y) + (res ? "_add" : "") + "[" + i64(rows) + "x" + i64(dim) + "]");
    return p.done(it::launch_rmsnorm_forward(ctx->stream, dtype_y == IT_BF16, rows, dim, eps, x, res, gamma,
                                             sum_out, y));
}

it_status it_rmsnorm_backward(it_context *ctx, int64_t rows, int64_t dim, float eps, const float *dy,
                              const float *x, const float *gamma, const float *gres, float *dx, float *dgamma) {
    if (!ctx) return fail(IT_ERR_NULL, "rmsnorm_backward: ctx is NULL");
    if (rows < 0 || dim < 0) return fail(IT_ERR_INVALID, "rmsnorm_backward: negative size");
    if (dim > 2048)
        return fail(IT_ERR_DIMS, "rmsnorm_backward: unsupported dimensions, dim must be at most 2048, got " + i64(dim));
    if (dim == 0) return IT_OK;
    if (!dgamma || !gamma) return fail(IT_ERR_NULL, "rmsnorm_backward: NULL buffer");
    if (rows == 0) return it::launch_zero(ctx->stream, dgamma, (size_t)dim * sizeof(float));
    if (!dy || !x || !dx) return fail(IT_ERR_NULL, "rmsnorm_backward: NULL buffer");
    void *part = nullptr;
    if (const it_status st = it::ensure_scratch(ctx, (size_t)it::rmsnorm_backward_scratch_bytes(rows, dim), &part);
        st != IT_OK)
        return st;
    Prof p(ctx, std::string("rmsnorm_bwd") + (gres ? "_add" : "") + "[" + i64(rows) + "x" + i64(dim) + "]");
    return p.done(it::launch_rmsnorm_backward(ctx->stream, rows, dim, eps, dy, x, gamma, gres, dx, dgamma,
                                              (float *)part));
}

it_status it_fused_rmsnorm_linear(it_context *ctx, int64_t rows, int64_t hidden, int64_t out_features, float eps,
                                  const float *input, const float *gamma, const float *weight, float *out) {
    if (!ctx) return fail(IT_ERR_NULL, "fused_rmsnorm_linear: ctx is NULL");
    if (rows < 0 || hidden < 0 || out_features < 0) return fail(IT_ERR_INVALID, "fused_rmsnorm_linear: negative size");
    if (rows == 0 || out_features == 0) return IT_OK;
    if (!out) return fail(IT_ERR_NULL, "fused_rmsnorm_linear: NULL buffer");
    if (hidden == 0) return it::launch_zero(ctx->stream, out, (size_t)(rows * out_features) * sizeof(float));
    if (!input || !gamma || !weight) return fail(IT_ERR_NULL, "fused_rmsnorm_linear: NULL buffer");
    it::GemmArgs a{};
    a.A = input;
    a.B = weight;
    a.C = out;
    a.M = rows;
    a.N = out_features;
    a.K = hidden;
    a.lda = hidden;
    a.ldb = hidden;
    a.ldc = out_features;
    a.batch_inner = 1;
    a.batch = 1;
    a.alpha = 1.f;
    a.a_vec_ok = (uintptr_t)input % 16 == 0 && hidden % 4 == 0;
    a.b_vec_ok = (uintptr_t)weight % 16 == 0 && hidden % 4 == 0;
    a.c_vec_ok = (uintptr_t)out % 16 == 0 && out_features % 4 == 0;
    a.a_kscale = gamma;  // the kernel also sums each row's squares and applies 1/rms in its epilogue
    a.rms_eps = eps;
    a.no_split = 1;
    return it::launch_gemm(ctx, IT_F32, false, true, a, "");
}

namespace {

// One FP32 GEMM of the chunked fused linear + cross entropy (C = op(A).op(B) + beta C).
it_status flce_gemm(it_context *ctx, bool ta, bool tb, int64_t M, int64_t N, int64_t K, const float *A, int64_t lda,
                    const float *B, int64_t ldb, float *C, int64_t ldc, float beta) {
    it::GemmArgs a{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.batch_inner = 1;
    a.batch = 1;
    a.alpha = 1.f;
    a.beta = beta;
    a.a_vec_ok = (uintptr_t)A % 16 == 0 && lda % 4 == 0;
    a.b_vec_ok = (uintptr_t)B % 16 == 0 && ldb % 4 == 0;
    a.c_vec_ok = (uintptr_t)C % 16 == 0 && ldc % 4 == 0;
    return it::launch_gemm(ctx, IT_F32, ta, tb, a, "flce");
}

size_t up256(size_t b) { return (b + 255) & ~(size_t)255; }

}  // namespace

it_status it_fused_linear_cross_entropy(it_context *ctx, int64_t rows, int64_t hidden, int64_t vocab,
                                        const float *hidden_states, const float *weight, const int32_t *targets,
                                        float *losses, float *loss_mean, float *grad_hidden, float *grad_weight,
                                        int64_t chunk_bytes) {
    if (!ctx) return fail(IT_ERR_NULL, "fused_linear_cross_entropy: ctx is NULL");
    if (rows < 0 || hidden < 0 || vocab < 0) return fail(IT_ERR_INVALID, "fused_linear_cross_entropy: negative size");
    if (!loss_mean) return fail(IT_ERR_NULL, "fused_linear_cross_entropy: loss_mean is NULL");
    if (rows == 0 || vocab == 0 || hidden == 0) {
        // Nothing to average: zero loss and gradients (the reference returns zeros for an empty batch).
        if (const it_status st = it::launch_zero(ctx->stream, loss_mean, sizeof(float)); st != IT_OK) return st;
        if (losses && rows > 0)
            if (const it_status st = it::launch_zero(ctx->stream, losses, (size_t)rows * 4); st != IT_OK) return st;
        if (grad_hidden && rows * hidden > 0)
            if (const it_status st = it::launch_zero(ctx->stream, grad_hidden, (size_t)(rows * hidden) * 4); st != IT_OK)
                return st;
        if (grad_weight && vocab * hidden > 0)
            if (const it_status st = it::launch_zero(ctx->stream, grad_weight, (size_t)(vocab * hidden) * 4);
                st != IT_OK)
                return st;
        return IT_OK;
    }
    if (!hidden_states || !weight || !targets) return fail(IT_ERR_NULL, "fused_linear_cross_entropy: NULL buffer");
    if (grad_weight && !grad_hidden)
        return fail(IT_ERR_INVALID, "fused_linear_cross_entropy: grad_weight needs grad_hidden");
    if (rows > 0x7fffffff) return fail(IT_ERR_DIMS, "fused_linear_cross_entropy: too many rows");
    // Vocabulary chunk: as many columns as fit the budget (default 256 MiB of logits), a multiple of
    // 128 (whole GEMM tiles) unless the vocabulary is smaller.
    const int64_t budget = chunk_bytes > 0 ? chunk_bytes : (int64_t)256 << 20;
    int64_t vc = budget / (rows * 4);
    vc = vc >= vocab ? vocab : std::max<int64_t>(128, vc / 128 * 128);
    if (vc > vocab) vc = vocab;
    const int64_t nchunks = (vocab + vc - 1) / vc;
    const size_t chunk_sz = up256((size_t)(rows * vc) * 4), stats_sz = up256((size_t)(rows * nchunks) * 8);
    const size_t row_sz = up256((size_t)rows * 4);
    void *ws = nullptr;
    if (const it_status st = it::ensure_attn_scratch(ctx, chunk_sz + stats_sz + 4 * row_sz + 256, &ws); st != IT_OK)
        return st;
    char *w8 = (char *)ws;
    float *chunk = (float *)w8;
    void *stats = w8 + chunk_sz;
    float *tlogit = (float *)(w8 + chunk_sz + stats_sz);
    float *lse = (float *)(w8 + chunk_sz + stats_sz + row_sz);
    float *loss_rows = losses ? losses : (float *)(w8 + chunk_sz + stats_sz + 2 * row_sz);
    float *scale = (float *)(w8 + chunk_sz + stats_sz + 3 * row_sz);
    auto v0_of = [&](int64_t c) { return c * vc; };
    auto vc_of = [&](int64_t c) { return std::min(vc, vocab - c * vc); };
    // Pass 1: logits chunk by chunk -> per-row (max, sum exp) and the target logit.
    for (int64_t c = 0; c < nchunks; ++c) {
        const int64_t v0 = v0_of(c), n = vc_of(c);
        if (const it_status st = flce_gemm(ctx, false, true, rows, n, hidden, hidden_states, hidden,
                                           weight + v0 * hidden, hidden, chunk, vc, 0.f);
            st != IT_OK)
            return st;
        Prof p(ctx, "flce_stats[" + i64(rows) + "x" + i64(n) + "]");
        if (const it_status st = p.done(it::launch_flce_chunk_stats(ctx->stream, chunk, vc, rows, n, v0, targets, vocab,
                                                                    stats, nchunks, c, tlogit));
            st != IT_OK)
            return st;
    }
    {
        Prof p(ctx, "flce_combine[" + i64(rows) + "x" + i64(nchunks) + "]");
        if (const it_status st = p.done(it::launch_flce_combine(ctx->stream, stats, nchunks, tlogit, targets, vocab,
                                                                rows, lse, loss_rows, loss_mean, scale));
            st != IT_OK)
            return st;
    }
    if (!grad_hidden) return IT_OK;
    // Pass 2, last chunk first (still in the buffer), then the others recomputed: the gradient
    // softmax - onehot in place, dW rows of the chunk (unscaled, as the reference), dH accumulated in
    // this fixed chunk order and scaled by 1 / valid count at the end.
    for (int64_t c = nchunks - 1; c >= 0; --c) {
        const int64_t v0 = v0_of(c), n = vc_of(c);
        if (c != nchunks - 1)
            if (const it_status st = flce_gemm(ctx, false, true, rows, n, hidden, hidden_states, hidden,
                                               weight + v0 * hidden, hidden, chunk, vc, 0.f);
                st != IT_OK)
                return st;
        {
            Prof p(ctx, "flce_grad[" + i64(rows) + "x" + i64(n) + "]");
            if (const it_status st =
                    p.done(it::launch_flce_chunk_grad(ctx->stream, chunk, vc, rows, n, v0, targets, vocab, lse));
                st != IT_OK)
                return st;
        }
        if (grad_weight)
            if (const it_status st = flce_gemm(ctx, true, false, n, hidden, rows, chunk, vc, hidden_states, hidden,
                                               grad_weight + v0 * hidden, hidden, 0.f);
                st != IT_OK)
                return st;
        if (const it_status st = flce_gemm(ctx, false, false, rows, hidden, n, chunk, vc, weight + v0 * hidden, hidden,
                                           grad_hidden, hidden, c == nchunks - 1 ? 0.f : 1.f);
            st != IT_OK)
            return st;
    }
    Prof p(ctx, "flce_scale[" + i64(rows) + "x" + i64(hidden) + "]");
    return p.done(it::launch_scale_by_device(ctx->stream, grad_hidden, rows * hidden, scale));
}

it_status it_rope(it_context *ctx, it_dtype dtype_src, it_dtype dtype_dst, int64_t batch, int64_t seq,
                  int64_t heads, int64_t head_dim, float base, int64_t position_offset, int backward,
                  const void *src, int64_t src_row_stride, void *dst, int64_t dst_row_stride, int64_t copy_cols) {
    if (!ctx) return fail(IT_ERR_NULL, "rope: ctx is NULL");
    if (!f32_or_bf16(dtype_src) || !f32_or_bf16(dtype_dst))
        return fail(IT_ERR_PRECISION, "rope: precision mismatch, expected FP32 or BF16");
    if (batch < 0 || seq < 0 || heads < 0 || head_dim < 0 || copy_cols < 0 || position_offset < 0)
        return fail(IT_ERR_INVALID, "rope: negative size");
    if (head_dim % 2 != 0) return fail(IT_ERR_SHAPE, "rope: head_dim must be even, got " + i64(head_dim));
    const int64_t width = heads * head_dim + copy_cols;
    if (src_row_stride < width || dst_row_stride < width)
        return fail(IT_ERR_SHAPE, "rope: row stride smaller than the rotated and copied columns");
    if (batch * seq == 0 || width == 0) return IT_OK;
    if (!src || !dst) return fail(IT_ERR_NULL, "rope: NULL buffer");
    if (src == dst && (dtype_src != dtype_dst || src_row_stride != dst_row_stride))
        return fail(IT_ERR_INVALID, "rope: in place needs the same precision and row stride");
    if (batch * seq > 0x7fffffff) return fail(IT_ERR_DIMS, "rope: too many rows");
    if (seq * (head_dim / 2) > 0x7fffffff) return fail(IT_ERR_DIMS, "rope: table too large");
    const void *table = nullptr;
    if (head_dim > 0)
        if (const it_status st = it::rope_table(ctx, seq, head_dim, base, position_offset, &table); st != IT_OK)
            return st;
    Prof p(ctx, std::string(backward ? "rope_bwd" : "rope_fwd") + sfx(dtype_dst) + "[" + i64(batch * seq) + "x" +
                    i64(heads) + "x" + i64(head_dim) + "]");
    return p.done(it::launch_rope(ctx->stream, dtype_src == IT_BF16, dtype_dst == IT_BF16, batch, seq, heads,
                                  head_dim, table, backward ? 1 : 0, src, src_row_stride, dst, dst_row_stride,
                                  src == dst ? 0 : copy_cols));
}

it_status it_embedding_forward(it_context *ctx, it_dtype dtype_table, it_dtype dtype_out, int64_t n, int64_t dim,
                               int64_t vocab, const void *table, const uint32_t *ids, void *out) {
    if (!ctx) return fail(IT_ERR_NULL, "embedding: ctx is NULL");
    if (!f32_or_bf16(dtype_table) || !f32_or_bf16(dtype_out))
        return fail(IT_ERR_PRECISION, "embedding: precision mismatch, expected FP32 or BF16");
    if (n < 0 || dim < 0 || vocab < 0) return fail(IT_ERR_INVALID, "embedding: negative size");
    if (n == 0 || dim == 0) return IT_OK;
    if (!table || !ids || !out) return fail(IT_ERR_NULL, "embedding: NULL buffer");
    Prof p(ctx, std::string("embedding_fwd") + sfx(dtype_out) + "[" + i64(n) + "x" + i64(dim) + "]");
    return p.done(it::launch_embedding_forward(ctx->stream, dtype_table == IT_BF16, dtype_out == IT_BF16, n, dim,
                                               vocab, table, ids, out));
}

it_status it_embedding_backward(it_context *ctx, int64_t n, int64_t dim, int64_t vocab, const float *dy,
                                const uint32_t *ids, float *dw) {
    if (!ctx) return fail(IT_ERR_NULL, "embedding_backward: ctx is NULL");
    if (n < 0 || dim < 0 || vocab < 0) return fail(IT_ERR_INVALID, "embedding_backward: negative size");
    if (vocab == 0 || dim == 0) return IT_OK;
    if (!dw) return fail(IT_ERR_NULL, "embedding_backward: NULL buffer");
    if (n == 0) return it::launch_zero(ctx->stream, dw, (size_t)(vocab * dim) * sizeof(float));
    if (!dy || !ids) return fail(IT_ERR_NULL, "embedding_backward: NULL buffer");
    if ((vocab + 15) / 16 > 0x7fffffff) return fail(IT_ERR_DIMS, "embedding_backward: vocabulary too large");
    Prof p(ctx, "embedding_bwd[" + i64(n) + "x" + i64(dim) + ",V=" + i64(vocab) + "]");
    return p.done(it::launch_embedding_backward(ctx->stream, n, dim, vocab, dy, ids, dw));
}

it_status it_cross_entropy_fused(it_context *ctx, it_dtype dtype_grad, int64_t rows, int64_t vocab,
                                 const float *logits, const uint32_t *targets, float *losses, void *grad,
                                 float *loss_mean) {
    if (!ctx) return fail(IT_ERR_NULL, "cross_entropy_fused: ctx is NULL");
    if (!f32_or_bf16(dtype_grad))
        return fail(IT_ERR_PRECISION, "cross_entropy_fused: precision mismatch, expected FP32 or BF16");
    if (rows < 0 || vocab < 0) return fail(IT_ERR_INVALID, "cross_entropy_fused: negative size");
    if (rows > 0x7fffffff) return fail(IT_ERR_DIMS, "cross_entropy_fused: too many rows");
    if (rows == 0) {
        // The reference returns a zero loss for an empty batch.
        return loss_mean ? it::launch_zero(ctx->stream, loss_mean, sizeof(float)) : IT_OK;
    }
    if (vocab == 0) return fail(IT_ERR_SHAPE, "cross_entropy_fused: vocabulary is empty");
    if (!logits || !targets || !grad) return fail(IT_ERR_NULL, "cross_entropy_fused: NULL buffer");
    if (!losses) {
        void *p = nullptr;
        if (const it_status st = it::ensure_scratch(ctx, (size_t)rows * sizeof(float), &p); st != IT_OK) return st;
        losses = (float *)p;
    }
    const bool vec_ok = vocab % 4 == 0 && (uintptr_t)logits % 16 == 0 &&
                        (uintptr_t)grad % (dtype_grad == IT_BF16 ? 8 : 16) == 0;
    Prof p(ctx, std::string("cross_entropy") + sfx(dtype_grad) + "[" + i64(rows) + "x" + i64(vocab) + "]");
    return p.done(it::launch_cross_entropy(ctx->stream, dtype_grad == IT_BF16, rows, vocab, logits, targets, losses,
                                           grad, nullptr, loss_mean, vec_ok));
}

it_status it_cross_entropy_stats(it_context *ctx, int64_t rows, int64_t vocab, const float *logits,
                                 const uint32_t *targets, float *losses, float *stats, float *loss_mean) {
    if (!ctx) return fail(IT_ERR_NULL, "cross_entropy_stats: ctx is NULL");
    if (rows < 0 || vocab < 0) return fail(IT_ERR_INVALID, "cross_entropy_stats: negative size");
    if (rows > 0x7fffffff) return fail(IT_ERR_DIMS, "cross_entropy_stats: too many rows");
    if (rows == 0) return loss_mean ? it::launch_zero(ctx->stream, loss_mean, sizeof(float)) : IT_OK;
    if (vocab == 0) return fail(IT_ERR_SHAPE, "cross_entropy_stats: vocabulary is empty");
    if (!logits || !targets || !stats) return fail(IT_ERR_NULL, "cross_entropy_stats: NULL buffer");
    if ((uintptr_t)stats % 8 != 0) return fail(IT_ERR_INVALID, "cross_entropy_stats: stats must be 8-byte aligned");
    if (!losses) {
        void *p = nullptr;
        if (const it_status st = it::ensure_scratch(ctx, (size_t)rows * sizeof(float), &p); st != IT_OK) return st;
        losses = (float *)p;
    }
    const bool vec_ok = vocab % 4 == 0 && (uintptr_t)logits % 16 == 0;
    Prof p(ctx, "cross_entropy_stats[" + i64(rows) + "x" + i64(vocab) + "]");
    return p.done(it::launch_cross_entropy(ctx->stream, false, rows, vocab, logits, targets, losses, nullptr, stats,
                                           loss_mean, vec_ok));
}

it_status it_swiglu_backward(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, int64_t rows, int64_t cols,
                             const float *grad_out, int64_t ld_grad, const void *gate, const void *up,
                             int64_t ld_in, void *grad_gate, void *grad_up, int64_t ld_out) {
    if (!ctx) return fail(IT_ERR_NULL, "swiglu_backward: ctx is NULL");
    if (!f32_or_bf16(dtype_in) || !f32_or_bf16(dtype_out))
        return fail(IT_ERR_PRECISION, "swiglu_backward: precision mismatch, expected FP32 or BF16");
    if (rows < 0 || cols < 0) return fail(IT_ERR_INVALID, "swiglu_backward: negative size");
    if (ld_grad < cols || ld_in < cols || ld_out < cols)
        return fail(IT_ERR_SHAPE, "swiglu_backward: leading dimension smaller than cols");
    if (rows == 0 || cols == 0) return IT_OK;
    if (rows > 0x7fffffff) return fail(IT_ERR_DIMS, "swiglu_backward: too many rows");
    if (!grad_out || !gate || !up || !grad_gate || !grad_up) return fail(IT_ERR_NULL, "swiglu_backward: NULL buffer");
    Prof p(ctx, std::string("swiglu_bwd") + sfx(dtype_out) + "[" + i64(rows) + "x" + i64(cols) + "]");
    return p.done(it::launch_swiglu_backward(ctx->stream, dtype_in == IT_BF16, dtype_out == IT_BF16, rows, cols,
                                             grad_out, ld_grad, gate, up, ld_in, grad_gate, grad_up, ld_out));
}

it_status it_grad_norm_clip(it_context *ctx, int count, const float *const *grads, const int64_t *sizes,
                            float max_norm, float *out) {
    if (!ctx) return fail(IT_ERR_NULL, "total_l2_norm: ctx is NULL");
    if (count < 0) return fail(IT_ERR_INVALID, "total_l2_norm: negative count");
    if (!out) return fail(IT_ERR_NULL, "total_l2_norm: NULL output");
    if (count > 0 && (!grads || !sizes)) return fail(IT_ERR_NULL, "total_l2_norm: NULL table");
    for (int i = 0; i < count; ++i) {
        if (sizes[i] < 0) return fail(IT_ERR_INVALID, "total_l2_norm: negative size");
        if (sizes[i] > 0 && !grads[i]) return fail(IT_ERR_NULL, "total_l2_norm: NULL buffer");
    }
    const int64_t parts = it::grad_norm_partials(count, sizes);
    void *part = nullptr;
    if (const it_status st = it::ensure_scratch(ctx, (size_t)(parts > 0 ? parts : 1) * sizeof(double), &part);
        st != IT_OK)
        return st;
    Prof p(ctx, "grad_norm[" + std::to_string(count) + " tensors]");
    return p.done(it::launch_grad_norm(ctx->stream, count, grads, sizes, max_norm, out, (double *)part));
}

it_status it_lion_step(it_context *ctx, int count, float *const *weights, float *const *momentum,
                       const float *const *grads, const int64_t *sizes, float lr, float beta1, float beta2,
                       float weight_decay, const float *grad_scale, const float *lr_dev) {
    if (!ctx) return fail(IT_ERR_NULL, "lion: ctx is NULL");
    if (count < 0) return fail(IT_ERR_INVALID, "lion: negative count");
    if (count == 0) return IT_OK;
    if (!weights || !momentum || !grads || !sizes) return fail(IT_ERR_NULL, "lion: NULL table");
    for (int i = 0; i < count; ++i) {
        if (sizes[i] < 0) return fail(IT_ERR_INVALID, "lion: negative size");
        if (sizes[i] > 0 && (!weights[i] || !momentum[i] || !grads[i])) return fail(IT_ERR_NULL, "lion: NULL buffer");
    }
    Prof p(ctx, "lion[" + std::to_string(count) + " tensors]");
    return p.done(it::launch_lion(ctx->stream, count, weights, momentum, grads, sizes, lr, beta1, beta2, weight_decay,
                                  grad_scale, lr_dev));
}

}  // extern "C"
