// C ABI entry points for the contractions: argument validation (the reference's TensorError cases,
// src/ops/mps_gemm.rs:45-108,439-452), GEMM dispatch, precision conversion, and the attention
// forward / backward compositions (src/ops/attention.rs:286-377, src/train/helpers.rs:120-193).
#include <cmath>
#include <cstdint>
#include <string>
#include <vector>

#include "internal.hpp"

using it::fail;

namespace {

const char *dtype_name(it_dtype d) {
    switch (d) {
    case IT_F32: return "FP32";
    case IT_F16: return "FP16";
    case IT_BF16: return "BF16";
    }
    return "unknown";
}

// 4 consecutive output elements per store: 16 B for f32, 8 B for bf16.
bool out_vec_ok(const void *p, bool bf16, int64_t ld, int64_t s1, int64_t s2) {
    const uintptr_t align = bf16 ? 8 : 16;
    return ((uintptr_t)p % align == 0) && ld % 4 == 0 && s1 % 4 == 0 && s2 % 4 == 0;
}

bool vec_ok(const void *p, int elem_bytes, int64_t ld, int64_t s1, int64_t s2) {
    const int64_t vec = 16 / elem_bytes;
    return ((uintptr_t)p % 16 == 0) && ld % vec == 0 && s1 % vec == 0 && s2 % vec == 0;
}

std::string i64(int64_t v) { return std::to_string((long long)v); }

}  // namespace

extern "C" {

it_status it_gemm_check(it_dtype dtype_in, it_dtype dtype_out, it_op transA, it_op transB,
                        int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, int64_t strideA,
                        const void *B, int64_t ldb, int64_t strideB, float beta, const void *C,
                        int64_t ldc, int64_t strideC, int64_t batch, const it_epilogue *epi) {
    if (dtype_in != IT_F32 && dtype_in != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string("matmul: precision mismatch, expected FP32 or BF16, got ") +
                                          dtype_name(dtype_in));
    if (dtype_out != IT_F32 && dtype_out != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string("matmul: precision mismatch, expected FP32 or BF16 output, got ") +
                                          dtype_name(dtype_out));
    if ((transA != IT_OP_N && transA != IT_OP_T) || (transB != IT_OP_N && transB != IT_OP_T))
        return fail(IT_ERR_INVALID, "matmul: transA/transB must be IT_OP_N or IT_OP_T");
    if (M < 0 || N < 0 || K < 0 || batch < 0)
        return fail(IT_ERR_INVALID, "matmul: negative size (M=" + i64(M) + ", N=" + i64(N) +
                                        ", K=" + i64(K) + ", batch=" + i64(batch) + ")");
    const int64_t min_lda = transA == IT_OP_T ? M : K;
    const int64_t min_ldb = transB == IT_OP_T ? K : N;
    if (lda < (min_lda > 1 ? min_lda : 1))
        return fail(IT_ERR_INVALID, "matmul: lda " + i64(lda) + " < " + i64(min_lda));
    if (ldb < (min_ldb > 1 ? min_ldb : 1))
        return fail(IT_ERR_INVALID, "matmul: ldb " + i64(ldb) + " < " + i64(min_ldb));
    const bool swb = epi && (epi->flags & IT_EPI_SWIGLU_BWD);
    const int64_t min_ldc = swb ? 2 * N : N;
    if (ldc < (min_ldc > 1 ? min_ldc : 1)) return fail(IT_ERR_INVALID, "matmul: ldc " + i64(ldc) + " < " + i64(min_ldc));
    if (strideA < 0 || strideB < 0 || strideC < 0)
        return fail(IT_ERR_INVALID, "matmul: negative batch stride");
    const bool has_out = M > 0 && N > 0 && batch > 0;
    if (has_out && !C) return fail(IT_ERR_NULL, "matmul: C is NULL");
    if (has_out && K > 0 && (!A || !B)) return fail(IT_ERR_NULL, "matmul: A or B is NULL");
    if (epi) {
        const uint32_t known =
            IT_EPI_BIAS | IT_EPI_SWIGLU | IT_EPI_CAUSAL | IT_EPI_ROPE | IT_EPI_SWIGLU_BWD | IT_EPI_XENT_A;
        if (epi->flags & ~known) return fail(IT_ERR_INVALID, "matmul: unknown epilogue flags");
        if ((epi->flags & IT_EPI_BIAS) && !epi->bias)
            return fail(IT_ERR_NULL, "matmul: bias epilogue without a bias pointer");
        if (epi->flags & IT_EPI_SWIGLU) {
            if (!epi->B2 && has_out && K > 0)
                return fail(IT_ERR_NULL, "matmul: SwiGLU epilogue without B2");
            if (transA != IT_OP_N || transB != IT_OP_T)
                return fail(IT_ERR_INVALID, "matmul: SwiGLU epilogue needs transA=N, transB=T (Y = X.W^T)");
            if (epi->flags & IT_EPI_CAUSAL)
                return fail(IT_ERR_INVALID, "matmul: SwiGLU epilogue cannot be combined with causal");
        }
        if ((epi->flags & (IT_EPI_SWIGLU | IT_EPI_CAUSAL)) && beta != 0.f)
            return fail(IT_ERR_INVALID, "matmul: beta != 0 cannot be combined with SwiGLU or causal");
        if (epi->flags & IT_EPI_SWIGLU_BWD) {
            if (epi->flags != IT_EPI_SWIGLU_BWD)
                return fail(IT_ERR_INVALID, "matmul: the SwiGLU-backward epilogue combines with no other flag");
            if (beta != 0.f) return fail(IT_ERR_INVALID, "matmul: beta != 0 cannot be combined with SwiGLU backward");
            if (has_out && (!epi->gate_out || !epi->up_out))
                return fail(IT_ERR_NULL, "matmul: SwiGLU-backward epilogue without gate or up");
            if (batch > 1) return fail(IT_ERR_INVALID, "matmul: SwiGLU backward is a single (unbatched) product");
        }
        if (epi->flags & IT_EPI_XENT_A) {
            if (epi->flags != IT_EPI_XENT_A)
                return fail(IT_ERR_INVALID, "matmul: the cross-entropy operand combines with no other flag");
            if (dtype_in != IT_F32)
                return fail(IT_ERR_PRECISION, "matmul: the cross-entropy operand needs FP32 inputs");
            if (transB != IT_OP_N) return fail(IT_ERR_INVALID, "matmul: the cross-entropy operand needs transB=N");
            if (batch > 1) return fail(IT_ERR_INVALID, "matmul: the cross-entropy operand is a single (unbatched) product");
            if (has_out && K > 0 && (!epi->xent_stats || !epi->xent_targets))
                return fail(IT_ERR_NULL, "matmul: cross-entropy operand without stats or targets");
            if ((uintptr_t)epi->xent_stats % 8 != 0)
                return fail(IT_ERR_INVALID, "matmul: cross-entropy stats must be 8-byte aligned");
        }
        if (epi->flags & IT_EPI_ROPE) {
            if (epi->flags & (IT_EPI_SWIGLU | IT_EPI_CAUSAL))
                return fail(IT_ERR_INVALID, "matmul: RoPE cannot be combined with SwiGLU or causal");
            if (epi->rope_head_dim <= 0 || epi->rope_head_dim % 2 != 0 || epi->rope_seq <= 0 ||
                epi->rope_cols < 0 || epi->rope_cols > N || epi->rope_cols % epi->rope_head_dim != 0 ||
                epi->rope_offset < 0)
                return fail(IT_ERR_INVALID, "matmul: bad RoPE parameters");
            if (N % 4 != 0 || ldc % 4 != 0 || (C && (uintptr_t)C % 16 != 0))
                return fail(IT_ERR_DIMS, "matmul: RoPE epilogue needs N % 4 == 0 and a 16-byte aligned C with ldc % 4 == 0");
        }
    }
    return IT_OK;
}

// The kernel arguments of one it_gemm call (already validated).
static it_status gemm_args(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, int64_t M, int64_t N, int64_t K,
                           float alpha, const void *A, int64_t lda, int64_t strideA, const void *B, int64_t ldb,
                           int64_t strideB, float beta, void *C, int64_t ldc, int64_t strideC, int64_t batch,
                           const it_epilogue *epi, it::GemmArgs &a) {
    const int eb = dtype_in == IT_BF16 ? 2 : 4;
    a = it::GemmArgs{};
    a.A = A;
    a.B = B;
    a.C = C;
    a.M = M;
    a.N = N;
    a.K = K;
    a.lda = lda;
    a.ldb = ldb;
    a.ldc = ldc;
    a.sA_in = strideA;
    a.sB_in = strideB;
    a.sC_in = strideC;
    a.batch_inner = batch;
    a.batch = batch;
    a.alpha = alpha;
    a.beta = beta;
    a.out_bf16 = dtype_out == IT_BF16;
    a.a_vec_ok = vec_ok(A, eb, lda, strideA, 0);
    a.b_vec_ok = vec_ok(B, eb, ldb, strideB, 0);
    a.c_vec_ok = out_vec_ok(C, a.out_bf16, ldc, strideC, 0);
    if (epi) {
        a.has_bias = (epi->flags & IT_EPI_BIAS) != 0;
        a.bias = epi->bias;
        if (epi->flags & IT_EPI_SWIGLU) {
            a.dual = 1;
            a.B2 = epi->B2;
            a.G = epi->gate_out;
            a.U = epi->up_out;
            // The pre-activations are stored with C's vector width when all three allow it.
            a.c_vec_ok = a.c_vec_ok && (!a.G || out_vec_ok(a.G, a.out_bf16, ldc, strideC, 0)) &&
                         (!a.U || out_vec_ok(a.U, a.out_bf16, ldc, strideC, 0));
            a.b_vec_ok = a.b_vec_ok && vec_ok(epi->B2, eb, ldb, strideB, 0);
        }
        if (epi->flags & IT_EPI_CAUSAL) {
            a.causal = it::CAUSAL_WRITE;
            a.causal_offset = epi->causal_offset;
        }
        if (epi->flags & IT_EPI_SWIGLU_BWD) {
            a.swiglu_bwd = 1;
            a.G = epi->gate_out;
            a.U = epi->up_out;
            const uintptr_t al = a.out_bf16 ? 8 : 16;
            a.c_vec_ok = a.c_vec_ok && N % 4 == 0 && (uintptr_t)a.G % al == 0 && (uintptr_t)a.U % al == 0;
        }
        if (epi->flags & IT_EPI_XENT_A) {
            a.xent_stats = (const float2 *)epi->xent_stats;
            a.xent_tgt = epi->xent_targets;
            a.xent_scale = epi->xent_scale;
        }
        if (epi->flags & IT_EPI_ROPE) {
            const void *table = nullptr;
            if (const it_status rs = it::rope_table(ctx, epi->rope_seq, epi->rope_head_dim, epi->rope_base,
                                                    epi->rope_offset, &table);
                rs != IT_OK)
                return rs;
            a.rope_table = (const float2 *)table;
            a.rope_seq = epi->rope_seq;
            a.rope_half = (int)(epi->rope_head_dim / 2);
            a.rope_cols = epi->rope_cols;
        }
    }
    return IT_OK;
}

it_status it_gemm(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, it_op transA, it_op transB,
                  int64_t M, int64_t N, int64_t K, float alpha,
                  const void *A, int64_t lda, int64_t strideA,
                  const void *B, int64_t ldb, int64_t strideB,
                  float beta, void *C, int64_t ldc, int64_t strideC,
                  int64_t batch, const it_epilogue *epi) {
    it_status st = it_gemm_check(dtype_in, dtype_out, transA, transB, M, N, K, A, lda, strideA, B,
                                 ldb, strideB, beta, C, ldc, strideC, batch, epi);
    if (st != IT_OK) return st;
    if (!ctx) return fail(IT_ERR_NULL, "matmul: ctx is NULL");
    if (M == 0 || N == 0 || batch == 0) return IT_OK;
    it::GemmArgs a;
    st = gemm_args(ctx, dtype_in, dtype_out, M, N, K, alpha, A, lda, strideA, B, ldb, strideB, beta, C, ldc, strideC,
                   batch, epi, a);
    if (st != IT_OK) return st;
    return it::launch_gemm(ctx, dtype_in, transA == IT_OP_T, transB == IT_OP_T, a, "");
}

it_status it_gemm_group(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, int count,
                        const it_gemm_call *calls) {
    if (count < 0 || count > 8) return fail(IT_ERR_INVALID, "matmul group: count must be 0..8, got " + i64(count));
    if (count > 0 && !calls) return fail(IT_ERR_NULL, "matmul group: calls is NULL");
    for (int i = 0; i < count; ++i) {
        const it_gemm_call &c = calls[i];
        const it_status st = it_gemm_check(dtype_in, dtype_out, c.transA, c.transB, c.M, c.N, c.K, c.A, c.lda,
                                           c.strideA, c.B, c.ldb, c.strideB, c.beta, c.C, c.ldc, c.strideC, c.batch,
                                           c.epi);
        if (st != IT_OK) return st;
    }
    // One launch may run the calls concurrently: no call's outputs may touch another call's
    // operands or outputs (byte ranges, strides included; broadcast operands count once).
    struct Range {
        uintptr_t lo, hi;
    };
    auto extent = [](const void *p, int64_t batch, int64_t stride, int64_t rows, int64_t ld, int64_t cols,
                     int64_t eb) {
        const uintptr_t lo = (uintptr_t)p;
        return Range{lo, lo + (uintptr_t)(((batch - 1) * stride + (rows - 1) * ld + cols) * eb)};
    };
    const int64_t eb_in = dtype_in == IT_BF16 ? 2 : 4, eb_out = dtype_out == IT_BF16 ? 2 : 4;
    std::vector<Range> outs[8], ins[8];
    for (int i = 0; i < count; ++i) {
        const it_gemm_call &c = calls[i];
        if (c.M == 0 || c.N == 0 || c.batch == 0) continue;
        const uint32_t fl = c.epi ? c.epi->flags : 0u;
        const int64_t cols = (fl & IT_EPI_SWIGLU_BWD) ? 2 * c.N : c.N;
        outs[i].push_back(extent(c.C, c.batch, c.strideC, c.M, c.ldc, cols, eb_out));
        if ((fl & IT_EPI_SWIGLU) && c.epi->gate_out)
            outs[i].push_back(extent(c.epi->gate_out, c.batch, c.strideC, c.M, c.ldc, c.N, eb_out));
        if ((fl & IT_EPI_SWIGLU) && c.epi->up_out)
            outs[i].push_back(extent(c.epi->up_out, c.batch, c.strideC, c.M, c.ldc, c.N, eb_out));
        if (c.K > 0) {
            const bool ta = c.transA == IT_OP_T, tb = c.transB == IT_OP_T;
            ins[i].push_back(extent(c.A, c.batch, c.strideA, ta ? c.K : c.M, c.lda, ta ? c.M : c.K, eb_in));
            ins[i].push_back(extent(c.B, c.batch, c.strideB, tb ? c.N : c.K, c.ldb, tb ? c.K : c.N, eb_in));
            if ((fl & IT_EPI_SWIGLU) && c.epi->B2)
                ins[i].push_back(extent(c.epi->B2, c.batch, c.strideB, tb ? c.N : c.K, c.ldb, tb ? c.K : c.N, eb_in));
        }
    }
    for (int i = 0; i < count; ++i)
        for (int j = 0; j < count; ++j) {
            if (i == j) continue;
            for (const Range &o : outs[i]) {
                auto hit = [&](const std::vector<Range> &v) {
                    for (const Range &r : v)
                        if (o.lo < r.hi && r.lo < o.hi) return true;
                    return false;
                };
                if (hit(ins[j]) || hit(outs[j]))
                    return fail(IT_ERR_INVALID, "matmul group: the output of call " + i64(i) +
                                                    " overlaps the operands or outputs of call " + i64(j));
            }
        }
    if (!ctx) return fail(IT_ERR_NULL, "matmul: ctx is NULL");
    // Empty GEMMs are skipped; the library groups the rest where it pays.
    it::GemmArgs args[8];
    bool ta[8], tb[8];
    int n = 0;
    for (int i = 0; i < count; ++i) {
        const it_gemm_call &c = calls[i];
        if (c.M == 0 || c.N == 0 || c.batch == 0) continue;
        ta[n] = c.transA == IT_OP_T;
        tb[n] = c.transB == IT_OP_T;
        const it_status st = gemm_args(ctx, dtype_in, dtype_out, c.M, c.N, c.K, c.alpha, c.A, c.lda, c.strideA, c.B,
                                       c.ldb, c.strideB, c.beta, c.C, c.ldc, c.strideC, c.batch, c.epi, args[n]);
        if (st != IT_OK) return st;
        ++n;
    }
    return it::launch_gemm_group(ctx, dtype_in, ta, tb, args, n, "");
}

it_status it_f32_to_bf16(it_context *ctx, const float *src, uint16_t *dst, int64_t n) {
    if (!ctx) return fail(IT_ERR_NULL, "to_bf16_gpu: ctx is NULL");
    if (n < 0) return fail(IT_ERR_INVALID, "to_bf16_gpu: negative length");
    if (n == 0) return IT_OK;
    if (!src || !dst) return fail(IT_ERR_NULL, "to_bf16_gpu: NULL buffer");
    return it::launch_f32_to_bf16(ctx->stream, src, dst, n);
}

it_status it_bf16_to_f32(it_context *ctx, const uint16_t *src, float *dst, int64_t n) {
    if (!ctx) return fail(IT_ERR_NULL, "to_f32_gpu: ctx is NULL");
    if (n < 0) return fail(IT_ERR_INVALID, "to_f32_gpu: negative length");
    if (n == 0) return IT_OK;
    if (!src || !dst) return fail(IT_ERR_NULL, "to_f32_gpu: NULL buffer");
    return it::launch_bf16_to_f32(ctx->stream, src, dst, n);
}

it_status it_softmax_rows(it_context *ctx, const float *S, void *P, it_dtype dtype_p,
                          int64_t batch, int64_t rows, int64_t cols, int causal,
                          int64_t causal_offset) {
    if (!ctx) return fail(IT_ERR_NULL, "softmax: ctx is NULL");
    if (dtype_p != IT_F32 && dtype_p != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string("softmax: precision mismatch, expected FP32 or BF16, got ") +
                                          dtype_name(dtype_p));
    if (batch < 0 || rows < 0 || cols < 0) return fail(IT_ERR_INVALID, "softmax: negative size");
    if (batch * rows * cols == 0) return IT_OK;
    if (!S || !P) return fail(IT_ERR_NULL, "softmax: NULL buffer");
    return it::launch_softmax_rows(ctx->stream, S, P, dtype_p == IT_BF16, batch, rows, cols,
                                   causal != 0, causal_offset, rows * cols, rows * cols);
}

it_status it_softmax_backward(it_context *ctx, const float *dY, const void *Y, it_dtype dtype_y,
                              void *dX, it_dtype dtype_dx, int64_t batch, int64_t rows,
                              int64_t cols, int causal) {
    if (!ctx) return fail(IT_ERR_NULL, "softmax_backward: ctx is NULL");
    if ((dtype_y != IT_F32 && dtype_y != IT_BF16) || (dtype_dx != IT_F32 && dtype_dx != IT_BF16))
        return fail(IT_ERR_PRECISION, "softmax_backward: precision mismatch, expected FP32 or BF16");
    if (batch < 0 || rows < 0 || cols < 0) return fail(IT_ERR_INVALID, "softmax_backward: negative size");
    if (batch * rows * cols == 0) return IT_OK;
    if (!dY || !Y || !dX) return fail(IT_ERR_NULL, "softmax_backward: NULL buffer");
    return it::launch_softmax_backward(ctx->stream, dY, Y, dtype_y == IT_BF16, dX,
                                       dtype_dx == IT_BF16, batch, rows, cols, causal != 0);
}

it_status it_transpose_3d(it_context *ctx, const float *in, float *out, int64_t batch, int64_t m, int64_t n) {
    if (!ctx) return fail(IT_ERR_NULL, "transpose_3d_gpu: ctx is NULL");
    if (batch < 0 || m < 0 || n < 0) return fail(IT_ERR_INVALID, "transpose_3d_gpu: negative size");
    if (batch == 0 || m == 0 || n == 0) return IT_OK;
    if (!in || !out) return fail(IT_ERR_NULL, "transpose_3d_gpu: NULL buffer");
    const uintptr_t bytes = (uintptr_t)(batch * m * n) * sizeof(float);
    if ((uintptr_t)in < (uintptr_t)out + bytes && (uintptr_t)out < (uintptr_t)in + bytes)
        return fail(IT_ERR_INVALID, "transpose_3d_gpu: output overlaps the input");
    return it::launch_transpose_3d(ctx->stream, in, out, batch, m, n);
}

it_status it_causal_mask_3d(it_context *ctx, const float *in, float *out, int64_t batch, int64_t seq) {
    if (!ctx) return fail(IT_ERR_NULL, "causal_mask_3d_gpu: ctx is NULL");
    if (batch < 0 || seq < 0) return fail(IT_ERR_INVALID, "causal_mask_3d_gpu: negative size");
    if (batch == 0 || seq == 0) return IT_OK;
    if (!in || !out) return fail(IT_ERR_NULL, "causal_mask_3d_gpu: NULL buffer");
    const uintptr_t bytes = (uintptr_t)(batch * seq * seq) * sizeof(float);
    if (in != out && (uintptr_t)in < (uintptr_t)out + bytes && (uintptr_t)out < (uintptr_t)in + bytes)
        return fail(IT_ERR_INVALID, "causal_mask_3d_gpu: output partially overlaps the input");
    return it::launch_causal_mask_3d(ctx->stream, in, out, batch, seq);
}

it_status it_fill_normal(it_context *ctx, it_dtype dtype, uint64_t seed, int64_t offset, int64_t n,
                         double std_dev, void *dst) {
    if (!ctx) return fail(IT_ERR_NULL, "fill_normal: ctx is NULL");
    if (dtype != IT_F32 && dtype != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string("fill_normal: precision mismatch, expected FP32 or BF16, got ") +
                                          dtype_name(dtype));
    if (n < 0 || offset < 0) return fail(IT_ERR_INVALID, "fill_normal: negative size or offset");
    if (n == 0) return IT_OK;
    if (!dst) return fail(IT_ERR_NULL, "fill_normal: dst is NULL");
    return it::launch_fill_normal(ctx->stream, dtype == IT_BF16, dst, seed, offset, n, std_dev);
}

}  // extern "C"

// ------------------------------------------------------------------ attention compositions

namespace {

struct AttnGeom {
    int64_t bh, Sq, Skv, D;
    it_attn_layout lay;     // Q, dQ
    it_attn_layout kv_lay;  // K, V, dK, dV
    it_attn_layout o_lay;   // O, dO
};

bool bad_layout(const it_attn_layout &l, int64_t head_dim) {
    return l.heads < 1 || l.row_stride < head_dim || l.batch_stride < 0 || l.head_stride < 0;
}

it_status check_attention(const char *op, it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq_q,
                          int64_t seq_kv, int64_t head_dim, const it_attn_layout *q_layout,
                          const it_attn_layout *kv_layout, const it_attn_layout *o_layout,
                          AttnGeom *g) {
    if (!ctx) return fail(IT_ERR_NULL, std::string(op) + ": ctx is NULL");
    if (dtype != IT_F32 && dtype != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string(op) + ": precision mismatch, expected FP32 or BF16, got " +
                                          dtype_name(dtype));
    if (bh < 0 || seq_q < 0 || seq_kv < 0 || head_dim < 0)
        return fail(IT_ERR_INVALID, std::string(op) + ": negative size");
    it_attn_layout lay{1, seq_q * head_dim, 0, head_dim};
    if (q_layout) lay = *q_layout;
    it_attn_layout kv{1, seq_kv * head_dim, 0, head_dim};
    if (kv_layout)
        kv = *kv_layout;
    else if (q_layout)
        kv = *q_layout;
    it_attn_layout ol = o_layout ? *o_layout : lay;
    if (bad_layout(lay, head_dim) || bad_layout(kv, head_dim) || bad_layout(ol, head_dim))
        return fail(IT_ERR_INVALID, std::string(op) + ": bad layout strides");
    if (bh % lay.heads != 0 || lay.heads != kv.heads || lay.heads != ol.heads)
        return fail(IT_ERR_SHAPE, std::string(op) + ": shape mismatch, expected batch*heads divisible by heads " +
                                      i64(lay.heads) + ", got " + i64(bh));
    *g = AttnGeom{bh, seq_q, seq_kv, head_dim, lay, kv, ol};
    return IT_OK;
}

// Base GEMM arguments for a [S or D] x [S or D] contraction over the BH batch, with the per-head
// operands addressed through the two-level layout and the [BH,S,S] workspaces contiguous.
it::GemmArgs attn_args(const AttnGeom &g, int64_t M, int64_t N, int64_t K, int eb) {
    it::GemmArgs a{};
    a.M = M;
    a.N = N;
    a.K = K;
    a.batch = g.bh;
    a.batch_inner = g.lay.heads;
    a.alpha = 1.f;
    (void)eb;
    return a;
}

struct Operand {
    const void *p;
    int64_t ld, s_in, s_out;
};

Operand q_operand(const AttnGeom &g, const void *p) {
    return Operand{p, g.lay.row_stride, g.lay.head_stride, g.lay.batch_stride};
}

Operand o_operand(const AttnGeom &g, const void *p) {
    return Operand{p, g.o_lay.row_stride, g.o_lay.head_stride, g.o_lay.batch_stride};
}

Operand kv_operand(const AttnGeom &g, const void *p) {
    return Operand{p, g.kv_lay.row_stride, g.kv_lay.head_stride, g.kv_lay.batch_stride};
}

// [BH, Sq, Skv] contiguous score-shaped workspace.
Operand score_operand(const AttnGeom &g, const void *p) {
    return Operand{p, g.Skv, g.Sq * g.Skv, g.lay.heads * g.Sq * g.Skv};
}

void set_A(it::GemmArgs &a, const Operand &o, int eb) {
    a.A = o.p;
    a.lda = o.ld;
    a.sA_in = o.s_in;
    a.sA_out = o.s_out;
    a.a_vec_ok = vec_ok(o.p, eb, o.ld, o.s_in, o.s_out);
}

void set_B(it::GemmArgs &a, const Operand &o, int eb) {
    a.B = o.p;
    a.ldb = o.ld;
    a.sB_in = o.s_in;
    a.sB_out = o.s_out;
    a.b_vec_ok = vec_ok(o.p, eb, o.ld, o.s_in, o.s_out);
}

void set_C(it::GemmArgs &a, const Operand &o, bool bf16_out) {
    a.C = const_cast<void *>(o.p);
    a.ldc = o.ld;
    a.sC_in = o.s_in;
    a.sC_out = o.s_out;
    a.out_bf16 = bf16_out;
    a.c_vec_ok = out_vec_ok(o.p, bf16_out, o.ld, o.s_in, o.s_out);
}

// Sc = scale * Q.K^T (causal tiles skipped), P = softmax(Sc).
it_status attn_scores(it_context *ctx, it_dtype dtype, const AttnGeom &g, float scale, int causal,
                      const void *Q, const void *K, float *Sc, void *P) {
    const int eb = dtype == IT_BF16 ? 2 : 4;
    it::GemmArgs a = attn_args(g, g.Sq, g.Skv, g.D, eb);
    set_A(a, q_operand(g, Q), eb);
    set_B(a, kv_operand(g, K), eb);
    set_C(a, score_operand(g, Sc), false);
    a.alpha = scale;
    a.causal = causal ? it::CAUSAL_SKIP : it::CAUSAL_NONE;
    it_status st = it::launch_gemm(ctx, dtype, false, true, a, "attn.S=QK^T");
    if (st != IT_OK) return st;
    return it::launch_softmax_rows(ctx->stream, Sc, P, dtype == IT_BF16, g.bh, g.Sq, g.Skv,
                                   causal != 0, 0, g.Sq * g.Skv, g.Sq * g.Skv);
}

}  // namespace

extern "C" {

it_status it_attention_forward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq_q,
                               int64_t seq_kv, int64_t head_dim, float scale, int causal,
                               const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                               const it_attn_layout *o_layout,
                               const void *Q, const void *K, const void *V,
                               float *Sc, void *P, float *O) {
    AttnGeom g;
    it_status st = check_attention("attention", ctx, dtype, bh, seq_q, seq_kv, head_dim, q_layout,
                                   kv_layout, o_layout, &g);
    if (st != IT_OK) return st;
    if (causal && seq_q != seq_kv)
        return fail(IT_ERR_SHAPE, "attention: shape mismatch, expected seq_q == seq_kv for causal, got " +
                                      i64(seq_q) + " and " + i64(seq_kv));
    if (bh == 0 || seq_q == 0 || head_dim == 0) return IT_OK;
    if (!Q || !O) return fail(IT_ERR_NULL, "attention: NULL buffer");
    const int eb = dtype == IT_BF16 ? 2 : 4;
    if (seq_kv > 0) {
        if (!K || !V || !Sc || !P) return fail(IT_ERR_NULL, "attention: NULL buffer");
        st = attn_scores(ctx, dtype, g, scale, causal, Q, K, Sc, P);
        if (st != IT_OK) return st;
    }
    // With seq_kv == 0 this GEMM has K = 0 and writes zeros (the reference returns zeros).
    // O = P.V (NN); with a causal P only k <= row contributes.
    it::GemmArgs a = attn_args(g, g.Sq, g.D, g.Skv, eb);
    set_A(a, score_operand(g, P), eb);
    set_B(a, kv_operand(g, V), eb);
    set_C(a, o_operand(g, O), false);
    a.kmode = causal ? it::KMODE_LOWER : it::KMODE_FULL;
    return it::launch_gemm(ctx, dtype, false, false, a, "attn.O=PV");
}

it_status it_attention_backward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                int64_t head_dim, float scale, int causal,
                                const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                const it_attn_layout *o_layout,
                                const void *dO, const void *Q, const void *K, const void *V,
                                float *Sc, void *P, float *dP, void *dS,
                                float *dQ, float *dK, float *dV) {
    AttnGeom g;
    it_status st = check_attention("attention_backward", ctx, dtype, bh, seq, seq, head_dim, q_layout,
                                   kv_layout, o_layout, &g);
    if (st != IT_OK) return st;
    if (bh == 0 || seq == 0 || head_dim == 0) return IT_OK;
    if (!dO || !Q || !K || !V || !Sc || !P || !dP || !dS || !dQ || !dK || !dV)
        return fail(IT_ERR_NULL, "attention_backward: NULL buffer");
    const int eb = dtype == IT_BF16 ? 2 : 4;
    st = attn_scores(ctx, dtype, g, scale, causal, Q, K, Sc, P);
    if (st != IT_OK) return st;

    // dV = P^T.dO (TN): op(A)[j][i] = P[i][j], nonzero only for i >= j under the causal mask.
    it::GemmArgs a = attn_args(g, g.Sq, g.D, g.Sq, eb);
    set_A(a, score_operand(g, P), eb);
    set_B(a, o_operand(g, dO), eb);
    set_C(a, kv_operand(g, dV), false);
    a.kmode = causal ? it::KMODE_UPPER : it::KMODE_FULL;
    if ((st = it::launch_gemm(ctx, dtype, true, false, a, "attn.dV=P^TdO")) != IT_OK) return st;

    // dP = dO.V^T (NT); above-diagonal tiles are never read.
    a = attn_args(g, g.Sq, g.Sq, g.D, eb);
    set_A(a, o_operand(g, dO), eb);
    set_B(a, kv_operand(g, V), eb);
    set_C(a, score_operand(g, dP), false);
    a.causal = causal ? it::CAUSAL_SKIP : it::CAUSAL_NONE;
    if ((st = it::launch_gemm(ctx, dtype, false, true, a, "attn.dP=dOV^T")) != IT_OK) return st;

    // dS = P * (dP - rowdot(dP, P))
    st = it::launch_softmax_backward(ctx->stream, dP, P, dtype == IT_BF16, dS, dtype == IT_BF16,
                                     g.bh, g.Sq, g.Sq, causal != 0);
    if (st != IT_OK) return st;

    // dQ = scale * dS.K (NN), dS lower-triangular under the mask.
    a = attn_args(g, g.Sq, g.D, g.Sq, eb);
    set_A(a, score_operand(g, dS), eb);
    set_B(a, kv_operand(g, K), eb);
    set_C(a, q_operand(g, dQ), false);
    a.alpha = scale;
    a.kmode = causal ? it::KMODE_LOWER : it::KMODE_FULL;
    if ((st = it::launch_gemm(ctx, dtype, false, false, a, "attn.dQ=dSK")) != IT_OK) return st;

    // dK = scale * dS^T.Q (TN)
    a = attn_args(g, g.Sq, g.D, g.Sq, eb);
    set_A(a, score_operand(g, dS), eb);
    set_B(a, q_operand(g, Q), eb);
    set_C(a, kv_operand(g, dK), false);
    a.alpha = scale;
    a.kmode = causal ? it::KMODE_UPPER : it::KMODE_FULL;
    return it::launch_gemm(ctx, dtype, true, false, a, "attn.dK=dS^TQ");
}

}  // extern "C"

// ------------------------------------------------------------------ fused (flash) attention

namespace {

it::FlashArgs flash_args(const AttnGeom &g, float scale, int causal) {
    it::FlashArgs f{};
    f.bh = g.bh;
    f.sq = g.Sq;
    f.skv = g.Skv;
    f.head_dim = g.D;
    f.heads = g.lay.heads;
    f.q_bs = g.lay.batch_stride;
    f.q_hs = g.lay.head_stride;
    f.q_rs = g.lay.row_stride;
    f.kv_bs = g.kv_lay.batch_stride;
    f.kv_hs = g.kv_lay.head_stride;
    f.kv_rs = g.kv_lay.row_stride;
    f.o_bs = f.do_bs = g.o_lay.batch_stride;
    f.o_hs = f.do_hs = g.o_lay.head_stride;
    f.o_rs = f.do_rs = g.o_lay.row_stride;
    f.scale = scale;
    f.causal = causal ? 1 : 0;
    return f;
}

std::string flash_key(const char *what, bool bf16, const AttnGeom &g, int causal) {
    return std::string(what) + (bf16 ? "_bf16" : "_f32") + (causal ? "_causal" : "") + "[bh=" + i64(g.bh) +
           ",sq=" + i64(g.Sq) + ",skv=" + i64(g.Skv) + "]";
}

// The fused kernels hold a 64-wide head in registers. Other head sizes up to the reference flash
// op's limit (src/ops/flash_attention.rs:98) run the materialised contractions, with their
// [BH, Sq, Skv] score buffers in library-owned scratch.
constexpr int64_t FLASH_MAX_HEAD_DIM = 128;

size_t round256(size_t b) { return (b + 255) / 256 * 256; }

it_status flash_head_dim_ok(const char *op, int64_t head_dim) {
    if (head_dim > FLASH_MAX_HEAD_DIM)
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, head_dim must be <= " +
                                     i64(FLASH_MAX_HEAD_DIM) + ", got " + i64(head_dim));
    return IT_OK;
}

// Checks scale for the fused kernels: the BF16 forward takes each row's maximum of the unscaled
// scores and scales it afterwards, which is the maximum of the scaled scores only for scale > 0.
it_status flash_scale_ok(const char *op, float scale) {
    if (!(scale > 0.f) || !std::isfinite(scale))
        return fail(IT_ERR_INVALID, std::string(op) + ": scale must be finite and > 0, got " + std::to_string(scale));
    return IT_OK;
}

// Output dtype of the fused entry points: FP32, or BF16 from the BF16 fused kernels (BF16 operands,
// head_dim 64).
it_status flash_out_dtype_ok(const char *op, it_dtype dtype, it_dtype out_dtype, int64_t head_dim) {
    if (out_dtype != IT_F32 && out_dtype != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string(op) + ": precision mismatch, expected FP32 or BF16 output, got " +
                                          dtype_name(out_dtype));
    if (out_dtype == IT_BF16 && dtype != IT_BF16)
        return fail(IT_ERR_PRECISION, std::string(op) + ": precision mismatch, a BF16 output needs BF16 operands, got " +
                                          dtype_name(dtype));
    if (out_dtype == IT_BF16 && head_dim != 64)
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, a BF16 output needs head_dim 64, got " +
                                     i64(head_dim));
    return IT_OK;
}

// A BF16 O is read 8 values (16 bytes) at a time by the backward's row pass.
bool o16_ok(const void *O, const it_attn_layout &l) {
    return (uintptr_t)O % 16 == 0 && l.batch_stride % 8 == 0 && l.head_stride % 8 == 0 && l.row_stride % 8 == 0;
}

}  // namespace

extern "C" {

it_status it_flash_attention_forward_ex(it_context *ctx, it_dtype dtype, it_dtype out_dtype, int64_t bh,
                                        int64_t seq_q, int64_t seq_kv, int64_t head_dim, float scale, int causal,
                                        const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                        const it_attn_layout *o_layout, const void *Q, const void *K,
                                        const void *V, void *O, float *lse) {
    AttnGeom g;
    it_status st = check_attention("flash_attention", ctx, dtype, bh, seq_q, seq_kv, head_dim, q_layout,
                                   kv_layout, o_layout, &g);
    if (st != IT_OK) return st;
    if ((st = flash_out_dtype_ok("flash_attention", dtype, out_dtype, head_dim)) != IT_OK) return st;
    if (causal && seq_q != seq_kv)
        return fail(IT_ERR_SHAPE, "flash_attention: shape mismatch, expected seq_q == seq_kv for causal, got " +
                                      i64(seq_q) + " and " + i64(seq_kv));
    if ((st = flash_head_dim_ok("flash_attention", head_dim)) != IT_OK) return st;
    if (head_dim != 64) {
        if (lse)
            return fail(IT_ERR_DIMS, "flash_attention: unsupported dimensions, lse is written for head_dim 64 "
                                     "only, got " + i64(head_dim));
        if (bh == 0 || seq_q == 0 || head_dim == 0) return IT_OK;
        if (seq_kv == 0)
            return fail(IT_ERR_DIMS, "flash_attention: unsupported dimensions, seq_kv == 0 needs head_dim 64, got " +
                                         i64(head_dim));
        // Materialised: Sc [BH,Sq,Skv] f32 then P in dtype, both in scratch.
        const size_t n = (size_t)bh * (size_t)seq_q * (size_t)seq_kv;
        const size_t eb = dtype == IT_BF16 ? 2 : 4;
        void *ws = nullptr;
        if ((st = it::ensure_attn_scratch(ctx, round256(n * 4) + n * eb, &ws)) != IT_OK) return st;
        float *sc = (float *)ws;
        void *p = (char *)ws + round256(n * 4);
        return it_attention_forward(ctx, dtype, bh, seq_q, seq_kv, head_dim, scale, causal, q_layout, kv_layout,
                                    o_layout, Q, K, V, sc, p, (float *)O);
    }
    if ((st = flash_scale_ok("flash_attention", scale)) != IT_OK) return st;
    if (bh == 0 || seq_q == 0) return IT_OK;
    if (!Q || !O || (seq_kv > 0 && (!K || !V))) return fail(IT_ERR_NULL, "flash_attention: NULL buffer");
    it::FlashArgs f = flash_args(g, scale, causal);
    f.Q = Q;
    // With seq_kv == 0 the kernel reads no key; give it a valid pointer to form addresses from.
    f.K = seq_kv > 0 ? K : Q;
    f.V = seq_kv > 0 ? V : Q;
    f.O = O;
    f.lse = lse;
    f.o_bf16 = out_dtype == IT_BF16;
    const int eb = dtype == IT_BF16 ? 2 : 4;
    if (!it::flash_supported(f, eb, false) || (f.o_bf16 && !o16_ok(O, g.o_lay)))
        return fail(IT_ERR_DIMS, "flash_attention: unsupported dimensions, operands must be 16-byte aligned "
                                 "with strides that are multiples of 16 bytes");
    hipEvent_t ev = nullptr;
    std::string key;
    if (ctx->profiling) {
        key = flash_key("flash_fwd", dtype == IT_BF16, g, causal);
        it::profile_begin(ctx, key, &ev);
    }
    st = it::launch_flash_fwd(ctx->stream, f, dtype == IT_BF16);
    if (ctx->profiling) it::profile_end(ctx, key, ev);
    return st;
}

it_status it_flash_attention_forward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq_q,
                                     int64_t seq_kv, int64_t head_dim, float scale, int causal,
                                     const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                     const it_attn_layout *o_layout, const void *Q, const void *K,
                                     const void *V, float *O, float *lse) {
    return it_flash_attention_forward_ex(ctx, dtype, IT_F32, bh, seq_q, seq_kv, head_dim, scale, causal, q_layout,
                                         kv_layout, o_layout, Q, K, V, O, lse);
}

}  // extern "C"

namespace {

// Validates a fused-backward call and fills its kernel arguments (everything but O, lse and dlt).
// *empty is set when there is nothing to compute.
it_status flash_bwd_args(const char *op, it_context *ctx, it_dtype dtype, it_dtype out_dtype, int64_t bh,
                         int64_t seq, int64_t head_dim, float scale, int causal, const it_attn_layout *q_layout,
                         const it_attn_layout *kv_layout, const it_attn_layout *o_layout, const void *dO,
                         const void *Q, const void *K, const void *V, const void *O, const float *lse, void *dQ,
                         void *dK, void *dV, AttnGeom *g, it::FlashArgs *f, bool *empty) {
    *empty = false;
    it_status st = check_attention(op, ctx, dtype, bh, seq, seq, head_dim, q_layout, kv_layout, o_layout, g);
    if (st != IT_OK) return st;
    if ((st = flash_out_dtype_ok(op, dtype, out_dtype, head_dim)) != IT_OK) return st;
    if (head_dim != 64)
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, head_dim must be 64, got " +
                                     i64(head_dim));
    if ((st = flash_scale_ok(op, scale)) != IT_OK) return st;
    if ((O == nullptr) != (lse == nullptr))
        return fail(IT_ERR_INVALID, std::string(op) + ": pass both O and lse, or neither");
    if (bh == 0 || seq == 0) {
        *empty = true;
        return IT_OK;
    }
    if (!dO || !Q || !K || !V || !dQ || !dK || !dV) return fail(IT_ERR_NULL, std::string(op) + ": NULL buffer");
    *f = flash_args(*g, scale, causal);
    f->Q = Q;
    f->K = K;
    f->V = V;
    f->dO = dO;
    f->dQ = dQ;
    f->dK = dK;
    f->dV = dV;
    f->grad_bf16 = out_dtype == IT_BF16;
    f->o_bf16 = O && out_dtype == IT_BF16;
    const int eb = dtype == IT_BF16 ? 2 : 4;
    if (!it::flash_supported(*f, eb, true))
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, operands must be 16-byte "
                                                   "aligned with strides that are multiples of 16 bytes");
    if (O && (f->o_bf16 ? !o16_ok(O, g->o_lay)
                        : ((uintptr_t)O % 16 != 0 || g->o_lay.batch_stride % 4 || g->o_lay.head_stride % 4 ||
                           g->o_lay.row_stride % 4)))
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, O must be 16-byte aligned "
                                                   "with strides that are multiples of 16 bytes");
    return IT_OK;
}

}  // namespace

extern "C" {

it_status it_flash_attention_backward_ex(it_context *ctx, it_dtype dtype, it_dtype out_dtype, int64_t bh,
                                         int64_t seq, int64_t head_dim, float scale, int causal,
                                         const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                         const it_attn_layout *o_layout, const void *dO, const void *Q,
                                         const void *K, const void *V, const void *O, const float *lse,
                                         void *dQ, void *dK, void *dV) {
    AttnGeom g;
    it::FlashArgs f;
    bool empty = false;
    it_status st;
    if (head_dim != 64) {
        const char *op = "flash_attention_backward";
        if ((st = check_attention(op, ctx, dtype, bh, seq, seq, head_dim, q_layout, kv_layout, o_layout, &g)) != IT_OK)
            return st;
        if ((st = flash_out_dtype_ok(op, dtype, out_dtype, head_dim)) != IT_OK) return st;
        if ((st = flash_head_dim_ok(op, head_dim)) != IT_OK) return st;
        if (O || lse)
            return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, O and lse are read for head_dim "
                                                       "64 only (pass NULL to recompute), got " + i64(head_dim));
        if (bh == 0 || seq == 0 || head_dim == 0) return IT_OK;
        // Materialised recompute: Sc, dP f32 and P, dS in dtype, [BH, seq, seq] each, in scratch.
        const size_t n = (size_t)bh * (size_t)seq * (size_t)seq;
        const size_t eb = dtype == IT_BF16 ? 2 : 4;
        const size_t f32b = round256(n * 4), lowb = round256(n * eb);
        void *ws = nullptr;
        if ((st = it::ensure_attn_scratch(ctx, 2 * f32b + 2 * lowb, &ws)) != IT_OK) return st;
        char *base = (char *)ws;
        return it_attention_backward(ctx, dtype, bh, seq, head_dim, scale, causal, q_layout, kv_layout, o_layout,
                                     dO, Q, K, V, (float *)base, base + f32b, (float *)(base + f32b + lowb),
                                     base + 2 * f32b + lowb, (float *)dQ, (float *)dK, (float *)dV);
    }
    st = flash_bwd_args("flash_attention_backward", ctx, dtype, out_dtype, bh, seq, head_dim, scale, causal,
                        q_layout, kv_layout, o_layout, dO, Q, K, V, O, lse, dQ, dK, dV, &g, &f, &empty);
    if (st != IT_OK || empty) return st;
    const size_t rows = (size_t)bh * (size_t)seq;
    // Workspace: when the forward is recomputed, O [rows, 64] and lse [rows]; then the row arrays
    // the backward's row pass writes for its dQ + dK/dV kernel, dlt [2 rows].
    const size_t bytes = rows * 4 * (O ? 2 : 64 + 1 + 2);
    void *ws = nullptr;
    if ((st = it::ensure_attn_scratch(ctx, bytes, &ws)) != IT_OK) return st;
    f.dlt = (float *)ws + (O ? 0 : rows * 65);
    const bool bf16 = dtype == IT_BF16;
    hipEvent_t ev = nullptr;
    std::string key;
    if (ctx->profiling) {
        key = flash_key(O ? "flash_bwd" : "flash_bwd_recompute", bf16, g, causal);
        it::profile_begin(ctx, key, &ev);
    }
    if (O) {
        f.O = const_cast<void *>(O);
        f.lse = const_cast<float *>(lse);
    } else {
        f.O = ws;  // 256-byte aligned, so its float4 stores are aligned; f32 (o_bf16 is 0)
        f.lse = (float *)ws + rows * 64;
        // Recomputed O is [bh, seq, 64] contiguous.
        f.o_bs = f.heads * seq * 64;
        f.o_hs = seq * 64;
        f.o_rs = 64;
        st = it::launch_flash_fwd(ctx->stream, f, bf16);
    }
    if (st == IT_OK) st = it::launch_flash_bwd(ctx->stream, f, bf16);
    if (ctx->profiling) it::profile_end(ctx, key, ev);
    return st;
}

it_status it_flash_attention_backward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                      int64_t head_dim, float scale, int causal,
                                      const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                      const it_attn_layout *o_layout, const void *dO, const void *Q,
                                      const void *K, const void *V, const float *O, const float *lse,
                                      float *dQ, float *dK, float *dV) {
    return it_flash_attention_backward_ex(ctx, dtype, IT_F32, bh, seq, head_dim, scale, causal, q_layout, kv_layout,
                                          o_layout, dO, Q, K, V, O, lse, dQ, dK, dV);
}

it_status it_flash_attention_backward_noalloc(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                              int64_t head_dim, float scale, int causal,
                                              const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                              const it_attn_layout *o_layout, const void *dO, const void *Q,
                                              const void *K, const void *V, const float *O, const float *lse,
                                              float *dQ, float *dK, float *dV) {
    const char *op = "flash_attention_backward_noalloc";
    // The static workspace holds two floats per query row (rowsum(dO * O), and the LSE in the form
    // the dK/dV part reads) for at most max_rows rows; checked first, so a call it cannot hold is
    // refused before anything else is looked at.
    const int64_t max_rows = (int64_t)(IT_NOALLOC_SCRATCH_BYTES / (2 * sizeof(float)));
    if (bh > 0 && seq > 0 && bh > max_rows / seq)
        return fail(IT_ERR_DIMS, std::string(op) + ": unsupported dimensions, bh * seq = " + i64(bh) + " * " +
                                     i64(seq) + " query rows exceed the " + i64(max_rows) +
                                     " rows of the static workspace");
    if (ctx && (!O || !lse))
        return fail(IT_ERR_NULL, std::string(op) + ": O and lse are required (the forward is not recomputed)");
    AttnGeom g;
    it::FlashArgs f;
    bool empty = false;
    it_status st = flash_bwd_args(op, ctx, dtype, IT_F32, bh, seq, head_dim, scale, causal, q_layout, kv_layout,
                                  o_layout, dO, Q, K, V, O, lse, dQ, dK, dV, &g, &f, &empty);
    if (st != IT_OK || empty) return st;
    void *ws = it::noalloc_scratch(ctx->device);
    if (!ws) return fail(IT_ERR_NO_DEVICE, std::string(op) + ": no static workspace on device " + i64(ctx->device));
    f.O = const_cast<float *>(O);
    f.lse = const_cast<float *>(lse);
    f.dlt = (float *)ws;  // every row the backward reads is written first by its row pass
    return it::launch_flash_bwd(ctx->stream, f, dtype == IT_BF16);
}

}  // extern "C"
