/*
 * irontensor_hip.h -- C ABI of the MI355X (gfx950) matmul path for IronTensor.
 *
 * This is the drop-in boundary that IronTensor's Rust ops API binds through `extern "C"` (a
 * build.rs that compiles this library with hipcc, one `extern "C"` block and thin wrappers in the ops
 * modules). Everything is plain pointers and sizes: no Rust, C++ or torch types cross it.
 *
 * Conventions
 *   - Every function returns it_status (0 == IT_OK). On failure a thread-local message is left in
 *     it_last_error(). Argument errors are detected before any device work is enqueued.
 *   - Matrices are row-major (IronTensor tensors are contiguous row-major, src/tensor.rs:11-302).
 *   - One context owns one HIP stream on one device. All work is stream-ordered on it; a context is
 *     not thread-safe (IronTensor's CommandBatch state is thread-local, src/command_batch.rs:49-53).
 *   - Device buffers come from it_malloc (a caching arena over hipMalloc) or any hipMalloc'd memory;
 *     the caller owns them. Library scratch (split-K partials) belongs to the context.
 *   - it_dtype values follow the reference's Precision enum order (src/precision.rs:1-6).
 */
#ifndef IRONTENSOR_HIP_H
#define IRONTENSOR_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* The enums have int as their underlying type in C++ as well (IT_ENUM_INT), so that any int a C
 * caller passes is a valid value there and is refused by the argument checks, not undefined. */
#ifdef __cplusplus
#define IT_ENUM_INT : int
#else
#define IT_ENUM_INT
#endif

typedef enum it_status IT_ENUM_INT {
    IT_OK = 0,
    IT_ERR_INNER_DIM = 1,   /* TensorError::InnerDimensionMismatch (src/error.rs:28-33) */
    IT_ERR_SHAPE = 2,       /* TensorError::ShapeMismatch (src/error.rs:9-14) */
    IT_ERR_PRECISION = 3,   /* TensorError::PrecisionMismatch (src/error.rs:22-27) */
    IT_ERR_DIMS = 4,        /* TensorError::UnsupportedDimensions (src/error.rs:15-21) */
    IT_ERR_INVALID = 5,     /* TensorError::InvalidValue (src/error.rs:38-42): bad enum, ld, flag */
    IT_ERR_NULL = 6,        /* a required pointer is NULL */
    IT_ERR_OOM = 7,         /* device allocation failed (reference panics, src/tensor.rs:71-74) */
    IT_ERR_NO_DEVICE = 8,   /* no HIP device / bad ordinal (reference panics, src/device.rs:18-20) */
    IT_ERR_HIP = 9,         /* any other HIP runtime error */
    IT_ERR_NOT_READY = 10   /* it_event_query: work not finished yet (not a failure) */
} it_status;

typedef enum it_dtype IT_ENUM_INT { IT_F32 = 0, IT_F16 = 1, IT_BF16 = 2 } it_dtype;
typedef enum it_op IT_ENUM_INT { IT_OP_N = 0, IT_OP_T = 1 } it_op;

typedef struct it_context it_context;
typedef struct it_event it_event;

/* ---------------------------------------------------------------- runtime (device.rs, command_batch.rs) */

/* Replaces MetalContext::new/global (src/device.rs:15-29): selects `device`, creates the stream. */
it_status it_init(int device, it_context **out_ctx);
/* Drains the stream, releases cached memory and the stream. */
it_status it_shutdown(it_context *ctx);
/* Thread-local message for the last failing call on this thread ("" if none). */
const char *it_last_error(void);
const char *it_status_string(it_status status);
/* Number of visible HIP devices (0 when none); never fails. */
int it_device_count(void);
/* Device name and compute-unit count, for reports. */
it_status it_device_info(it_context *ctx, char *name, size_t name_len, int *num_cus,
                         int *clock_khz);

/* Device memory (replaces per-op MTLBuffer allocation, src/tensor.rs:63-88, src/ops/kernel.rs:70-80). */
it_status it_malloc(it_context *ctx, size_t bytes, void **out_ptr);
it_status it_free(it_context *ctx, void *ptr);
/* Bytes currently handed out (gpu_memory_allocated, src/device.rs:43-71). */
size_t it_mem_allocated(it_context *ctx);
/* Bytes of library-owned scratch (split-K partial sums, attention workspaces), including blocks
 * retired while graphs that may use them are alive (see it_graph_launch). The reference allocates
 * per op and has no such pool. */
size_t it_mem_scratch(it_context *ctx);
/* Returns cached blocks to the device. */
it_status it_empty_cache(it_context *ctx);

/* Copies. h2d and d2d are stream-ordered; d2h blocks until the data is on the host (the reference's
 * as_f32_slice reads after a sync, src/tensor.rs:136-159). */
it_status it_memcpy_h2d(it_context *ctx, void *dst, const void *src, size_t bytes);
it_status it_memcpy_d2h(it_context *ctx, void *dst, const void *src, size_t bytes);
it_status it_memcpy_d2d(it_context *ctx, void *dst, const void *src, size_t bytes);
/* Zero-fill with a kernel (safe to capture in a graph; replaces Tensor::zeros' CPU memset). */
it_status it_zero(it_context *ctx, void *dst, size_t bytes);

/* CommandBatch::sync (src/command_batch.rs:191-207): waits for all work of the context. */
it_status it_stream_sync(it_context *ctx);
/* The HIP stream (hipStream_t) the context currently launches on, for callers that interoperate. */
void *it_stream(it_context *ctx);

/*
 * Overlap of independent work (no counterpart in the reference, whose CommandBatch orders all work
 * on one queue, src/command_batch.rs:174-390): between it_side_begin and it_side_end, launches go
 * to a second stream (default priority) that first waits for everything issued so far on the main
 * stream; the main stream continues concurrently. it_side_join makes the main stream wait for the
 * side work (it_stream_sync, reads to the host, frees and it_capture_end do so themselves). Each
 * stream has its own split-K / attention scratch. Used by the training-step driver to run weight
 * gradients beside the data-gradient chain; graph capture records the fork and join.
 */
it_status it_side_begin(it_context *ctx);
it_status it_side_end(it_context *ctx);
it_status it_side_join(it_context *ctx);
/* commit_async / is_async_complete / wait_for_completion (src/command_batch.rs:228-272). */
it_status it_event_create(it_context *ctx, it_event **out_ev);
it_status it_event_record(it_context *ctx, it_event *ev);
it_status it_event_query(it_event *ev);    /* IT_OK when complete, IT_ERR_NOT_READY otherwise */
it_status it_event_sync(it_event *ev);
it_status it_event_elapsed_ms(it_event *start, it_event *end, float *ms);
it_status it_event_destroy(it_event *ev);

/* ---------------------------------------------------------------- GEMM */

/* Epilogue flags (it_epilogue.flags). */
#define IT_EPI_BIAS 0x1u        /* C[m,n] += bias[n]            (Linear bias, src/nn/linear.rs:8-18) */
#define IT_EPI_SWIGLU 0x2u      /* dual-B: C = silu(op(A).op(B)) * (op(A).op(B2)) (ffn, elementwise.metal:100-115) */
#define IT_EPI_CAUSAL 0x4u      /* C[m,n] = -inf where n > m + causal_offset (attention.metal:186-207) */
#define IT_EPI_ROPE 0x8u        /* rotary embedding of columns n < rope_cols (src/ops/rope.rs:22) */
#define IT_EPI_SWIGLU_BWD 0x10u /* SwiGLU backward of the product (src/ops/backward/elementwise.rs:149) */
#define IT_EPI_XENT_A 0x20u     /* A = logits read as their cross-entropy gradient (src/ops/backward/loss.rs:248) */

typedef struct it_epilogue {
    uint32_t flags;
    const float *bias;      /* IT_EPI_BIAS: [N] f32; with IT_EPI_SWIGLU [2N]: gate bias, then up bias */
    const void *B2;         /* IT_EPI_SWIGLU: up-projection weight, same dtype/layout/ldb/strideB as B */
    void *gate_out;         /* IT_EPI_SWIGLU (optional): pre-activation gate, out dtype, ldc/strideC;
                               IT_EPI_SWIGLU_BWD (input): the forward's gate [M, N], out dtype, ld N */
    void *up_out;           /* IT_EPI_SWIGLU (optional): pre-activation up, likewise;
                               IT_EPI_SWIGLU_BWD (input): the forward's up [M, N], out dtype, ld N */
    int64_t causal_offset;  /* IT_EPI_CAUSAL: mask columns n > m + causal_offset */
    /* IT_EPI_ROPE: row m is position (m % rope_seq) + rope_offset of its sequence; columns
     * n < rope_cols form heads of rope_head_dim (even) whose pairs (2i, 2i+1) rotate by
     * position / rope_base^(2i / rope_head_dim), as it_rope does. Needs N % 4 == 0 and a 16-byte
     * aligned C with ldc % 4 == 0 (the rotation works on 4-column vectors). */
    float rope_base;
    int64_t rope_seq;
    int64_t rope_head_dim;
    int64_t rope_cols;
    int64_t rope_offset;
    /* IT_EPI_XENT_A (dtype_in IT_F32, transB == IT_OP_N, batch 1, no other flag): A holds FP32
     * logits [tokens, classes] and enters the product as the gradient it_cross_entropy_fused would
     * have written: element x of token t and class c as
     * (exp(x - xent_stats[2t]) * xent_stats[2t+1] - (c == xent_targets[t])) * xent_scale, with
     * {max, 1/sum} per token from it_cross_entropy_stats and xent_scale = 1/tokens for the mean
     * loss. transA == IT_OP_N: rows of op(A) are tokens (dL/dh = G.E); IT_OP_T: op(A) = A^T and k is
     * the token (dL/dE = G^T.h). The gradient tensor is never stored. */
    const float *xent_stats;
    const uint32_t *xent_targets;
    float xent_scale;
} it_epilogue;

/*
 * C[b] = alpha * op(A[b]) . op(B[b]) + beta * C[b]  (then the epilogue), for b in [0, batch).
 *   op(A) is [M,K]: transA == IT_OP_N -> A stored [M,K], lda >= K; IT_OP_T -> A stored [K,M], lda >= M.
 *   op(B) is [K,N]: transB == IT_OP_N -> B stored [K,N], ldb >= N; IT_OP_T -> B stored [N,K], ldb >= K.
 *   C stored [M,N], ldc >= N. stride* are element strides between batch matrices (0 = broadcast).
 * dtype_in IT_F32: FP32 MFMA; IT_BF16: BF16 MFMA with FP32 accumulation. dtype_out IT_F32 or IT_BF16
 * (RNE of the FP32 result, as bfloat(sum) in src/shaders/bf16_ops.metal:93).
 * Replaces MPSMatrixMultiplication with transposeLeft/transposeRight (src/ops/mps_gemm.rs:169-181,
 * :278-290, :390-402, :519-537) and every Metal GEMM kernel (src/shaders/gemm.metal,
 * src/shaders/backward/gemm.metal, src/shaders/bf16_ops.metal:25-122).
 * epi may be NULL. beta != 0 is not combined with IT_EPI_SWIGLU or IT_EPI_CAUSAL.
 * IT_EPI_SWIGLU_BWD: the product is dL/dh of h = silu(gate) * up; C (ldc >= 2N) receives
 * dgate in columns [0, N) and dup in [N, 2N) of each row (the [T, 2F] gate|up gradient the
 * projection's backward reads); combines with no other flag, beta == 0.
 */
it_status it_gemm(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, it_op transA, it_op transB,
                  int64_t M, int64_t N, int64_t K, float alpha,
                  const void *A, int64_t lda, int64_t strideA,
                  const void *B, int64_t ldb, int64_t strideB,
                  float beta, void *C, int64_t ldc, int64_t strideC,
                  int64_t batch, const it_epilogue *epi);

/* One GEMM of an it_gemm_group call: it_gemm's arguments after dtype_in and dtype_out. */
typedef struct it_gemm_call {
    it_op transA, transB;
    int64_t M, N, K;
    float alpha;
    const void *A;
    int64_t lda, strideA;
    const void *B;
    int64_t ldb, strideB;
    float beta;
    void *C;
    int64_t ldc, strideC;
    int64_t batch;
    const it_epilogue *epi;
} it_gemm_call;

/* `count` (<= 8) independent GEMMs with the same dtypes, stream-ordered on the context's stream as
 * `count` it_gemm calls would be, each validated as it_gemm validates (the first failure is
 * returned before anything is launched). No counterpart in the reference, whose CommandBatch
 * (src/command_batch.rs:166-181) gathers a step's dispatches into one command buffer but issues
 * each GEMM as its own dispatch; for callers holding several GEMMs at once (a layer's weight
 * gradients). Each run of consecutive calls of one layout can become one launch: BF16 GEMMs of
 * batch 1 on whole 256 x 256 tiles with a plain epilogue whose tiles fit one round of the GPU run
 * with K unsplit; FP32 GEMMs of batch 1 with a plain epilogue, N % 4 == 0, that it_gemm would run
 * on 64 x 64 tiles run at one split count for the run and one grouped split-K sum, when that is
 * priced below the separate calls. Grouped results can differ in the last bits from separate
 * calls (another split of K); everything else runs exactly as it_gemm would. No call's outputs
 * (C, and gate_out / up_out of IT_EPI_SWIGLU) may overlap another call's operands or outputs, as
 * byte ranges with the strides included (IT_ERR_INVALID otherwise, before anything is launched). */
it_status it_gemm_group(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, int count,
                        const it_gemm_call *calls);

/* Validates it_gemm's arguments without touching the device (same status and message as it_gemm). */
it_status it_gemm_check(it_dtype dtype_in, it_dtype dtype_out, it_op transA, it_op transB,
                        int64_t M, int64_t N, int64_t K, const void *A, int64_t lda, int64_t strideA,
                        const void *B, int64_t ldb, int64_t strideB, float beta, const void *C,
                        int64_t ldc, int64_t strideC, int64_t batch, const it_epilogue *epi);

/* ---------------------------------------------------------------- precision (src/ops/bf16_ops/precision.rs) */

/* to_bf16_gpu (precision.rs:15-46): RNE, NaN stays NaN. */
it_status it_f32_to_bf16(it_context *ctx, const float *src, uint16_t *dst, int64_t n);
/* to_f32_gpu (precision.rs:48-78): exact widening. */
it_status it_bf16_to_f32(it_context *ctx, const uint16_t *src, float *dst, int64_t n);

/* ---------------------------------------------------------------- attention contractions */

/*
 * Softmax over rows of an FP32 matrix (src/shaders/softmax.metal), optionally causal: columns
 * c > r + causal_offset are treated as -inf and written as 0. P may be FP32 or BF16 (dtype_p).
 * rows are grouped into `batch` matrices of `rows` x `cols` (row r of each matrix is its local row).
 */
it_status it_softmax_rows(it_context *ctx, const float *S, void *P, it_dtype dtype_p,
                          int64_t batch, int64_t rows, int64_t cols, int causal,
                          int64_t causal_offset);

/*
 * Softmax backward dX = Y * (dY - rowdot(dY, Y)) (src/shaders/backward/softmax.metal:22-45).
 * Y is FP32 or BF16 (dtype_y, the dtype P was stored in); dX is FP32 or BF16 (dtype_dx).
 * Causal: columns c > r are written as 0 without reading.
 */
it_status it_softmax_backward(it_context *ctx, const float *dY, const void *Y, it_dtype dtype_y,
                              void *dX, it_dtype dtype_dx, int64_t batch, int64_t rows,
                              int64_t cols, int causal);

/*
 * transpose_3d_gpu (src/ops/attention.rs:395-449, kernel transpose_3d_f32 in
 * src/shaders/attention.metal:163-182; re-exported at src/ops/mod.rs:21):
 * out[b, j, i] = in[b, i, j] for in [batch, m, n] f32 and out [batch, n, m] f32. The output must
 * not overlap the input (the reference always writes a new tensor). HBM-bound: 8 bytes per element.
 */
it_status it_transpose_3d(it_context *ctx, const float *in, float *out, int64_t batch, int64_t m, int64_t n);

/*
 * causal_mask_3d_gpu (src/ops/attention.rs:455-517, kernel causal_mask_3d_f32 in
 * src/shaders/attention.metal:186-207; re-exported at src/ops/mod.rs:21):
 * out[b, r, c] = c > r ? -inf : in[b, r, c] over [batch, seq, seq] f32. in == out masks in place;
 * masked elements are written without being read.
 */
it_status it_causal_mask_3d(it_context *ctx, const float *in, float *out, int64_t batch, int64_t seq);

/*
 * Per-head operand layout: element (bh, s, d) lives at
 *   (bh / heads) * batch_stride + (bh % heads) * head_stride + s * row_stride + d.
 * [B,H,S,D] contiguous: heads = 1, batch_stride = S*D, head_stride = 0, row_stride = D.
 * [B,S,H,D] contiguous: heads = H, batch_stride = S*H*D, head_stride = D, row_stride = H*D.
 * A NULL layout pointer means [B,H,S,D] contiguous.
 */
typedef struct it_attn_layout {
    int64_t heads;
    int64_t batch_stride;
    int64_t head_stride;
    int64_t row_stride;
} it_attn_layout;

/*
 * Forward attention contractions (ops::attention after its layout transposes,
 * src/ops/attention.rs:286-377): Sc = scale * Q.K^T (NT GEMM; causal tiles above the diagonal are
 * skipped), P = softmax(Sc) (causal: columns > row are 0), O = P.V (NN GEMM; causal: only k <= row).
 * Q: [BH, seq_q, D] through q_layout; K, V: [BH, seq_kv, D] through kv_layout (NULL = q_layout);
 * O: [BH, seq_q, D] f32 through o_layout (NULL = q_layout).
 * Sc: [BH, seq_q, seq_kv] f32 workspace; P: [BH, seq_q, seq_kv] of dtype.
 * dtype IT_F32: everything FP32. IT_BF16: Q, K, V and P are BF16 (FP32 accumulation).
 * causal requires seq_q == seq_kv (as the reference asserts, src/ops/attention.rs:346-350).
 */
it_status it_attention_forward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq_q,
                               int64_t seq_kv, int64_t head_dim, float scale, int causal,
                               const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                               const it_attn_layout *o_layout,
                               const void *Q, const void *K, const void *V,
                               float *Sc, void *P, float *O);

/*
 * attention_backward_recompute (src/train/helpers.rs:120-193) on [BH, seq, D] operands:
 * recompute Sc, P; dV = P^T.dO (TN); dP = dO.V^T (NT); dS = softmax_backward(dP, P);
 * dQ = scale * dS.K (NN); dK = scale * dS^T.Q (TN).
 * Q and dQ use q_layout; K, V, dK, dV use kv_layout (NULL = q_layout); dO uses o_layout
 * (NULL = q_layout). dQ, dK, dV are f32, so with dtype BF16 their layouts are read as f32 strides.
 * IT_F32: all FP32. IT_BF16: Q, K, V, dO BF16; Sc, dP FP32; P, dS BF16; dQ, dK, dV FP32.
 * Workspaces Sc, dP: [BH,S,S] f32; P, dS: [BH,S,S] of dtype.
 */
it_status it_attention_backward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                int64_t head_dim, float scale, int causal,
                                const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                const it_attn_layout *o_layout,
                                const void *dO, const void *Q, const void *K, const void *V,
                                float *Sc, void *P, float *dP, void *dS,
                                float *dQ, float *dK, float *dV);

/*
 * Fused ("flash") forms of the two calls above for head_dim 64: the same mathematics as
 * ops::attention and attention_backward_recompute (src/ops/attention.rs:286-377,
 * src/train/helpers.rs:120-193), with no [seq, seq] buffer. The softmax runs online over 64-key
 * blocks (running row max and sum), so results match the materialised form to rounding.
 *
 * Forward: O = softmax(scale * Q.K^T [causal]).V, layouts and dtypes as it_attention_forward.
 * lse (NULL allowed): [BH, seq_q] f32 row log-sum-exp of scale * Q.K^T, for the backward.
 * seq_kv == 0 gives O = 0 (the reference returns zeros).
 *
 * Backward: dQ, dK, dV as it_attention_backward. O ([BH, seq, 64] f32 through o_layout, as
 * written by the forward) and lse are the forward's outputs; pass both NULL to recompute them
 * into library workspace (which grows once per shape; not during capture). dK and dV are summed
 * per key block and dQ per query block, without atomics, so results are deterministic.
 * IT_BF16 rounds P and dS to BF16 before their MFMA, as the materialised form stores them.
 *
 * head_dim 64 runs the fused kernels, which need 16-byte aligned operands whose strides are
 * multiples of 16 bytes (IT_ERR_DIMS otherwise) and a finite scale > 0 (IT_ERR_INVALID).
 * Any other head_dim up to 128 (the limit of src/ops/flash_attention.rs:98; IT_ERR_DIMS above it)
 * runs the materialised contractions of it_attention_forward / it_attention_backward with their
 * [BH, seq_q, seq_kv] buffers in library-owned scratch (2 * bh * seq_q * seq_kv * sizeof(f32) for
 * the forward, twice that for the backward; grown once per shape, not during capture); there lse
 * must be NULL, the backward's O and lse must be NULL (it always recomputes), and the forward
 * needs seq_kv > 0. causal requires seq_q == seq_kv.
 * The reference's flash_attention(q, k, v, causal) on [batch, heads, seq, head_dim] FP32 tensors
 * (src/ops/flash_attention.rs:76-193, re-exported at src/ops/mod.rs:36) is
 * it_flash_attention_forward(ctx, IT_F32, batch * heads, seq, seq, head_dim, 1 / sqrt(head_dim),
 * causal, NULL, NULL, NULL, q, k, v, out, NULL).
 */
it_status it_flash_attention_forward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq_q,
                                     int64_t seq_kv, int64_t head_dim, float scale, int causal,
                                     const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                     const it_attn_layout *o_layout, const void *Q, const void *K,
                                     const void *V, float *O, float *lse);
it_status it_flash_attention_backward(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                      int64_t head_dim, float scale, int causal,
                                      const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                      const it_attn_layout *o_layout, const void *dO, const void *Q,
                                      const void *K, const void *V, const float *O, const float *lse,
                                      float *dQ, float *dK, float *dV);
/*
 * The two calls above with the output dtype chosen: out_dtype IT_F32 is them exactly; IT_BF16
 * (BF16 operands and head_dim 64 only: IT_ERR_PRECISION / IT_ERR_DIMS otherwise) writes O, and dQ,
 * dK, dV, as BF16 rounded to nearest even from the FP32 results, with the same element strides,
 * and the backward then reads a BF16 O (16-byte aligned, strides multiples of 8 elements). lse
 * stays FP32. This is the reference trainer's data path in BF16 mode, where the attention output
 * feeds the output projection and dQ / dK / dV feed the Q/K/V projections' backward
 * (src/train/forward.rs:138-146, src/train/backward.rs:100-147), without an FP32 round trip.
 */
it_status it_flash_attention_forward_ex(it_context *ctx, it_dtype dtype, it_dtype out_dtype, int64_t bh,
                                        int64_t seq_q, int64_t seq_kv, int64_t head_dim, float scale, int causal,
                                        const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                        const it_attn_layout *o_layout, const void *Q, const void *K,
                                        const void *V, void *O, float *lse);
it_status it_flash_attention_backward_ex(it_context *ctx, it_dtype dtype, it_dtype out_dtype, int64_t bh,
                                         int64_t seq, int64_t head_dim, float scale, int causal,
                                         const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                         const it_attn_layout *o_layout, const void *dO, const void *Q,
                                         const void *K, const void *V, const void *O, const float *lse,
                                         void *dQ, void *dK, void *dV);

/*
 * it_flash_attention_backward without any device allocation. No counterpart in the reference: it is
 * for callers that cannot allocate (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc). Same arguments, kernels and results as it_flash_attention_backward, except:
 *   - O and lse (the forward's outputs) are required, since the forward is not recomputed
 *     (IT_ERR_NULL otherwise);
 *   - its one workspace, two floats per query row (rowsum(dO * O) and the row's LSE in the form the
 *     dK/dV part reads; 8 bytes per row), lives in a static device array of
 *     IT_NOALLOC_SCRATCH_BYTES (8 MiB) that each GPU the library runs on holds until the process
 *     ends, so bh * seq may be at most 1048576 rows (IT_ERR_DIMS otherwise, before any device work);
 *   - every call on a GPU shares that GPU's array: calls that overlap on one GPU (other streams or
 *     contexts) race. The array keeps the last call's values and needs no clearing: each call
 *     writes every row before it reads it.
 * Calls no hipMalloc, hipFree or other allocating routine, and no profiler hooks.
 */
#define IT_NOALLOC_SCRATCH_BYTES (8u << 20)
it_status it_flash_attention_backward_noalloc(it_context *ctx, it_dtype dtype, int64_t bh, int64_t seq,
                                              int64_t head_dim, float scale, int causal,
                                              const it_attn_layout *q_layout, const it_attn_layout *kv_layout,
                                              const it_attn_layout *o_layout, const void *dO, const void *Q,
                                              const void *K, const void *V, const float *O, const float *lse,
                                              float *dQ, float *dK, float *dV);

/* ---------------------------------------------------------------- training-step ops
 *
 * The row and elementwise work between the contractions of one training step
 * (src/train/trainer/train_step.rs:39-460, src/train/forward.rs:79-212, src/train/backward.rs:21-177).
 * All buffers are device memory, row-major and contiguous unless a stride says otherwise; the
 * calls are stream-ordered like it_gemm. Reductions run in a fixed order (no float atomics), so
 * results are bit-for-bit repeatable. IT_BF16 outputs are rounded to nearest even.
 */

/* RMSNorm with an optional residual add in front. s = x + res (res NULL: s = x), written to
 * sum_out unless NULL; y = s * (1 / sqrt(mean(s^2) + eps)) * gamma in dtype_y. x, res, sum_out
 * [rows, dim] f32, gamma [dim] f32.
 * Replaces rmsnorm (src/ops/norm.rs:31) and the residual add before it
 * (ops::add, src/ops/elementwise.rs:276, at src/train/forward.rs:155,190). */
it_status it_rmsnorm_forward(it_context *ctx, it_dtype dtype_y, int64_t rows, int64_t dim, float eps,
                             const float *x, const float *res, const float *gamma, float *sum_out, void *y);

/* Fused RMSNorm + projection: out[r, o] = (sum_j (x[r,j] * gamma[j]) * W[o,j]) / sqrt(mean(x_r^2) + eps),
 * FP32; input [rows, hidden], gamma [hidden], weight [out_features, hidden] (the Linear layout),
 * out [rows, out_features]. The normalized activations are never written: gamma scales the A tile
 * on its way into the MFMA GEMM and 1/rms (one value per row, library scratch) scales the result.
 * Replaces fused_rmsnorm_linear (src/ops/fused_rmsnorm_linear.rs:73-205; kernel
 * src/shaders/fused_rmsnorm_linear.metal:42-114). */
it_status it_fused_rmsnorm_linear(it_context *ctx, int64_t rows, int64_t hidden, int64_t out_features, float eps,
                                  const float *input, const float *gamma, const float *weight, float *out);

/* Fused linear + cross entropy without the [rows, vocab] logits: logits = H.W^T are produced in
 * vocabulary chunks of at most chunk_bytes (<= 0: 256 MiB) by the MFMA GEMM, reduced to per-row
 * (max, sum exp), combined into the log-sum-exp; then each chunk (recomputed unless it is the last
 * one) becomes softmax - onehot in place and feeds grad_weight[v0:v0+n] = chunk^T.H and
 * grad_hidden += chunk.W[v0:v0+n]. H [rows, hidden] and W [vocab, hidden] FP32; targets device
 * int32, any value outside [0, vocab) (the reference's -100) ignored. Outputs: *loss_mean (device)
 * = mean loss over valid rows; losses [rows] (NULL: scratch); grad_hidden (NULL: forward only) =
 * gradient of the mean loss (scaled by 1 / valid count); grad_weight (NULL: skipped) UNSCALED, as
 * the reference's weight-gradient kernel leaves it (src/shaders/fused_linear_cross_entropy.metal:
 * 119-185). Deterministic (chunk order fixed). Replaces fused_linear_cross_entropy and
 * fused_linear_cross_entropy_forward_only (src/ops/fused_linear_cross_entropy.rs:79-242, :246-374). */
it_status it_fused_linear_cross_entropy(it_context *ctx, int64_t rows, int64_t hidden, int64_t vocab,
                                        const float *hidden_states, const float *weight, const int32_t *targets,
                                        float *losses, float *loss_mean, float *grad_hidden, float *grad_weight,
                                        int64_t chunk_bytes);

/* RMSNorm backward with the residual gradient added behind: dx = gres + dRMSNorm/dx . dy
 * (gres NULL: no add), dgamma[dim] = sum over rows of dy * x / rms (overwritten). dim <= 2048.
 * Replaces rmsnorm_backward (src/ops/backward/norm.rs:20) and add_tensors
 * (src/train/backward.rs:73,158). */
it_status it_rmsnorm_backward(it_context *ctx, int64_t rows, int64_t dim, float eps, const float *dy,
                              const float *x, const float *gamma, const float *gres, float *dx, float *dgamma);

/* Rotary embedding over rows (b, s) of [batch, seq, heads, head_dim] with row strides (elements):
 * pairs (2i, 2i+1) of each head rotate by (s + position_offset) / base^(2i/head_dim); backward != 0
 * applies the inverse (transposed) rotation. src == dst works in place (same dtype and stride);
 * otherwise copy_cols further columns after heads*head_dim are copied (e.g. V of a fused QKV
 * gradient changing precision). Replaces rope (src/ops/rope.rs:22) and rope_backward
 * (src/ops/backward/rope.rs:16). */
it_status it_rope(it_context *ctx, it_dtype dtype_src, it_dtype dtype_dst, int64_t batch, int64_t seq,
                  int64_t heads, int64_t head_dim, float base, int64_t position_offset, int backward,
                  const void *src, int64_t src_row_stride, void *dst, int64_t dst_row_stride, int64_t copy_cols);

/* out[i] = table[ids[i]] ([n, dim]); ids are device uint32. The reference asserts every id is
 * below vocab on the host (src/ops/embedding.rs:41-49); host mirrors do the same before upload,
 * and the kernel writes a zero row for an out-of-range id instead of reading out of bounds.
 * Replaces embedding (src/ops/embedding.rs:21). */
it_status it_embedding_forward(it_context *ctx, it_dtype dtype_table, it_dtype dtype_out, int64_t n, int64_t dim,
                               int64_t vocab, const void *table, const uint32_t *ids, void *out);
/* dw[vocab, dim] = scatter-add of dy rows by id, every element summed in token order (no
 * atomics); rows no id hits are zero. Replaces embedding_backward (src/ops/backward/embedding.rs:21). */
it_status it_embedding_backward(it_context *ctx, int64_t n, int64_t dim, int64_t vocab, const float *dy,
                                const uint32_t *ids, float *dw);

/* The forward half of it_cross_entropy_fused: losses (NULL: library scratch) and *loss_mean as
 * there, plus stats[2r] = max_c x_r[c] and stats[2r+1] = 1 / sum_c exp(x_r[c] - max) (8-byte
 * aligned); no gradient is written. A GEMM with IT_EPI_XENT_A rebuilds the gradient from these.
 * Replaces the loss half of cross_entropy_fused (src/ops/backward/loss.rs:248). */
it_status it_cross_entropy_stats(it_context *ctx, int64_t rows, int64_t vocab, const float *logits,
                                 const uint32_t *targets, float *losses, float *stats, float *loss_mean);

/* Fused softmax cross entropy over logits [rows, vocab] f32 and device uint32 targets:
 * losses[r] = logsumexp(x_r) - x_r[t_r] (losses NULL: library scratch), grad = (softmax - onehot)
 * / rows in dtype_grad, *loss_mean (device f32, NULL to skip) = mean of losses. Replaces
 * cross_entropy_fused (src/ops/backward/loss.rs:248; kernel src/shaders/loss.metal:91-131). */
it_status it_cross_entropy_fused(it_context *ctx, it_dtype dtype_grad, int64_t rows, int64_t vocab,
                                 const float *logits, const uint32_t *targets, float *losses, void *grad,
                                 float *loss_mean);

/* SwiGLU backward: grad_up = g * silu(gate), grad_gate = g * up * silu'(gate), with leading
 * dimensions so the two results can land in one [rows, 2*cols] gate|up buffer. grad_out f32,
 * gate/up in dtype_in, results in dtype_out. Replaces swiglu_backward
 * (src/ops/backward/elementwise.rs:149; src/shaders/backward/elementwise.metal:101-126). */
it_status it_swiglu_backward(it_context *ctx, it_dtype dtype_in, it_dtype dtype_out, int64_t rows, int64_t cols,
                             const float *grad_out, int64_t ld_grad, const void *gate, const void *up,
                             int64_t ld_in, void *grad_gate, void *grad_up, int64_t ld_out);

/* Global L2 norm of `count` f32 device tensors (host arrays of pointers and element counts),
 * summed in double in a fixed order, and the clip factor, written to device out[2] = {norm,
 * norm > max_norm ? max_norm / norm : 1}. Nothing is read back to the host. Replaces
 * total_l2_norm_gpu (src/ops/reduction.rs:94) and the clip rule of
 * src/train/trainer/train_step.rs:405-414. */
it_status it_grad_norm_clip(it_context *ctx, int count, const float *const *grads, const int64_t *sizes,
                            float max_norm, float *out);

/* Lion over `count` tensors in one launch per 24: g' = g * (*grad_scale) (NULL: 1);
 * u = beta2 m + (1-beta2) g'; m = beta1 m + (1-beta1) g'; w -= lr sign(u) + lr wd w, with lr read
 * from *lr_dev when lr_dev is not NULL (a schedule value updated between graph replays).
 * Replaces Lion::step (src/optim/lion/optimizer.rs:54-106; src/shaders/lion.metal lion_step_f32)
 * applied after scale_gradients_inplace (src/train/trainer/train_step.rs:410-414). */
it_status it_lion_step(it_context *ctx, int count, float *const *weights, float *const *momentum,
                       const float *const *grads, const int64_t *sizes, float lr, float beta1, float beta2,
                       float weight_decay, const float *grad_scale, const float *lr_dev);

/* ---------------------------------------------------------------- synthetic inputs */

/*
 * Seeded N(0, std_dev^2) fill for benchmark and test inputs; no counterpart in the reference,
 * whose benchmark draws unseeded host values (src/bin/benchmark.rs:110-113). dst[e] (e < n) is
 * normal number offset + e of `seed`: SplitMix64 output i = mix(seed + (i + 1) * 0x9E3779B97F4A7C15),
 * uniforms from its top 53 bits, (bits + 0.5) / 2^53, and Box-Muller over consecutive uniform
 * pairs (number 2p = r cos(2 pi u_{2p+1}), 2p + 1 = r sin(2 pi u_{2p+1}), r = sqrt(-2 ln u_{2p}))
 * in float64, times std_dev, rounded to FP32 (then RNE to BF16 for IT_BF16). The same stream as
 * the Python package's synth.normal; results agree bit for bit except where the device's float64
 * log/sin/cos and the host libm's differ by an ulp and that ulp moves the FP32 rounding.
 */
it_status it_fill_normal(it_context *ctx, it_dtype dtype, uint64_t seed, int64_t offset, int64_t n,
                         double std_dev, void *dst);

/* ---------------------------------------------------------------- graphs (launch-bound loops) */

typedef struct it_graph it_graph;

/* Starts capturing the context's stream into a HIP graph. Until it_capture_end, no call may need a
 * new device allocation (it fails with IT_ERR_INVALID instead): run the work once eagerly first. */
it_status it_capture_begin(it_context *ctx);
/* Ends the capture and instantiates the graph. */
it_status it_capture_end(it_context *ctx, it_graph **out_graph);
/* Replays the graph on the context's stream. A graph keeps the device addresses it was captured
 * with: the caller's buffers must outlive it; the library's own scratch does (a scratch block that a
 * later, larger eager call replaces is retired, not freed, while any graph of the context lives).
 * Replays are asynchronous like other stream work (the reference's commit_async,
 * src/command_batch.rs:228-272). A graph replays only on the context that captured it
 * (IT_ERR_INVALID otherwise). */
it_status it_graph_launch(it_context *ctx, it_graph *graph);
/* Waits for the context's streams, then destroys the graph; when it was the context's last live
 * graph, frees the scratch blocks retired meanwhile. A graph may also be destroyed after
 * it_shutdown of its context. */
it_status it_graph_destroy(it_graph *graph);

/* ---------------------------------------------------------------- profiling (src/profile) */

/* Shape-keyed per-launch GPU timing with hipEvents on the context's stream, mirroring
 * Profiler::record_matmul_shape (src/ops/mps_gemm.rs:22-30,84-88). enable=0 turns it off. */
it_status it_profiler_enable(it_context *ctx, int enable);
it_status it_profiler_reset(it_context *ctx);
/* Writes a JSON object {"<kernel>|<shape key>": {"calls": n, "total_ms": t}, ...} (syncs first).
 * Returns IT_ERR_INVALID with *needed set when buf_len is too small. */
it_status it_profiler_report(it_context *ctx, char *buf, size_t buf_len, size_t *needed);
/* The same launches as matmul statistics by shape, as Profiler::record_matmul_shape keys them
 * (src/ops/mps_gemm.rs:22-30,421-422; src/profile/report.rs:198-230): a JSON object
 * {"[4096,256]x[768,256]^T": {"count": n, "total_ms": t}, ...} over every GEMM launch, whatever
 * its plan: A as stored, "[M,K]" or "[K,M]^T", then "x", then B as stored, "[K,N]" or "[N,K]^T".
 * A grouped launch (it_gemm_group) counts once for each of its GEMMs, its time shared among them
 * in proportion to their FLOPs. Same buffer protocol as it_profiler_report. */
it_status it_profiler_report_shapes(it_context *ctx, char *buf, size_t buf_len, size_t *needed);

#ifdef __cplusplus
}
#endif
#endif /* IRONTENSOR_HIP_H */
