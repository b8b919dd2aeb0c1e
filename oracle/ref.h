/*
 * IronTensor matmul-path CPU ORACLE -- test infrastructure only.
 *
 * This is a plain-C restatement of the reference's CPU arithmetic for the matrix-multiplication
 * path (IronTensor has no library CPU GEMM; its "plain-Rust CPU f32 matmul" is the inline triple
 * loop inside its unit tests). It exists so that tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg can CHECK the HIP path; nothing in the product links or calls it.
 *
 * Arithmetic contract (identical to the Rust loops, which rustc never contracts into FMA):
 *   - f32 accumulator, initialised to 0.0f, products added in increasing k order;
 *   - a separate multiply then add (built with -ffp-contract=off, no fast-math);
 *   - BF16 values are widened exactly to f32 before the multiply.
 * Row-parallel threading keeps each output's accumulation order, so results are bit-identical to
 * the single-thread loop for any thread count.
 *
 * Pinning (what checks each function; see tests/test_oracle.py):
 *   ref_gemm_f32     reference KATs (gemm.rs, mps_gemm.rs, backward/gemm.rs tests), exact integer
 *                    products vs numpy int64, NT(A,B)==NN(A,B^T) bit-exactness, f64 brute force.
 *   ref_gemm_f64     numpy float64 matmul (independent implementation).
 *   ref_gemm_bf16    exact small-integer inputs vs numpy int64; equals ref_gemm_f32 on widened inputs.
 *   ref_f32_to_bf16  precision.rs tests, hand-computed RNE ties, numpy bit-level restatement.
 *   ref_attention_*  closed forms (Q=0 gives prefix means of V; one key gives V), causal rows of P
 *                    sum to 1, numpy float64 attention.
 *   ref_softmax_backward  finite-difference Jacobian of the softmax on tiny rows.
 *   ref_swiglu*      closed forms at g=0 and numpy float64, finite-difference derivative.
 */
#ifndef IRONTENSOR_ORACLE_REF_H
#define IRONTENSOR_ORACLE_REF_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* src/precision.rs:24-29: RNE by adding 0x7FFF + lsb, then truncating (NaN quirk kept). */
uint16_t ref_f32_to_bf16(float x);
/* src/precision.rs:33-35 */
float ref_bf16_to_f32(uint16_t x);
void ref_f32_to_bf16_n(const float *src, uint16_t *dst, int64_t n);
void ref_bf16_to_f32_n(const uint16_t *src, float *dst, int64_t n);

/*
 * C[b] = op(A[b]) . op(B[b]) for b in [0, batch), row-major storage.
 *   transA == 0: A stored [M,K] (lda >= K);  transA == 1: A stored [K,M] (lda >= M).
 *   transB == 0: B stored [K,N] (ldb >= N);  transB == 1: B stored [N,K] (ldb >= K).
 * NN follows src/ops/gemm.rs:336-350 and :370-384 (batched), src/ops/mps_gemm.rs:653-667;
 * NT follows src/ops/backward/gemm.rs:478-492; TN follows src/ops/backward/gemm.rs:494-508.
 */
void ref_gemm_f32(int transA, int transB, int64_t M, int64_t N, int64_t K,
                  const float *A, int64_t lda, int64_t strideA,
                  const float *B, int64_t ldb, int64_t strideB,
                  float *C, int64_t ldc, int64_t strideC, int64_t batch, int nthreads);

/* Same loop with a double accumulator over f32 inputs: the error-analysis tie-breaker. */
void ref_gemm_f64(int transA, int transB, int64_t M, int64_t N, int64_t K,
                  const float *A, int64_t lda, int64_t strideA,
                  const float *B, int64_t ldb, int64_t strideB,
                  double *C, int64_t ldc, int64_t strideC, int64_t batch, int nthreads);

/*
 * BF16 in, f32 accumulate: src/shaders/bf16_ops.metal:25-44 (gemm_bf16) and :98-122 (batched).
 * out_bf16 == 0 writes the f32 sum to C (float*); out_bf16 == 1 writes bfloat(sum) RNE (uint16_t*),
 * as the reference kernels do at bf16_ops.metal:43,93,121.
 */
void ref_gemm_bf16(int transA, int transB, int64_t M, int64_t N, int64_t K,
                   const uint16_t *A, int64_t lda, int64_t strideA,
                   const uint16_t *B, int64_t ldb, int64_t strideB,
                   void *C, int out_bf16, int64_t ldc, int64_t strideC, int64_t batch, int nthreads);

/* Y[m,n] += bias[n]: src/nn/linear.rs:8-18 (add_bias_broadcast). */
void ref_add_bias(float *Y, const float *bias, int64_t M, int64_t N);

/* h = silu(g) * u with silu(g) = g * (1/(1+exp(-g))): src/shaders/elementwise.metal:100-115. */
void ref_swiglu(const float *gate, const float *up, float *out, int64_t n);
/* src/shaders/backward/elementwise.metal:101-126. */
void ref_swiglu_backward(const float *grad_out, const float *gate, const float *up,
                         float *grad_gate, float *grad_up, int64_t n);

/*
 * Row softmax as in reference_attention (src/ops/attention.rs:580-588): max fold from -inf,
 * exp(x - max) summed in order, then exp(x - max) / sum.  In place over rows x cols.
 */
void ref_softmax_rows(float *X, int64_t rows, int64_t cols);

/* grad_x = y * (grad_y - dot(grad_y, y)) per row: src/shaders/backward/softmax.metal:22-45. */
void ref_softmax_backward(const float *grad_y, const float *y, float *grad_x,
                          int64_t rows, int64_t cols);

/*
 * reference_attention (src/ops/attention.rs:544-621): q,k,v,out are [B,S,H,D]; scale = 1/sqrt(D);
 * scores = dot * scale; causal sets k_pos > q_pos to -inf; softmax per row; out = P . V.
 */
void ref_attention_bshd(const float *q, const float *k, const float *v, float *out,
                        int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int causal,
                        int nthreads);

/*
 * Same computation on [BH,S,D] operands (the [B,H,S,D] layout of attention_backward_recompute),
 * with an explicit scale.  P (optional, [BH,S,S]) receives the softmax weights.
 */
void ref_attention_fwd_bhsd(const float *q, const float *k, const float *v, float *out, float *P,
                            int64_t bh, int64_t seq, int64_t head_dim, float scale, int causal,
                            int nthreads);

/*
 * attention_backward_recompute (src/train/helpers.rs:120-193) on [BH,S,D]:
 *   S = Q.K^T; S *= scale; causal -inf; P = softmax(S); dV = P^T.dO; dP = dO.V^T;
 *   dS = softmax_backward(dP, P); dQ = (dS.K) * scale; dK = (dS^T.Q) * scale.
 * Each matmul uses ref_gemm_f32's loop.
 */
void ref_attention_bwd_bhsd(const float *dO, const float *q, const float *k, const float *v,
                            float *dQ, float *dK, float *dV,
                            int64_t bh, int64_t seq, int64_t head_dim, float scale, int causal,
                            int nthreads);

/* Number of hardware threads the oracle would use by default (sysconf). */
int ref_default_threads(void);

/* ---- training-step ops around the contractions (train_ref.c) ----
 * Pinning (tests/test_oracle_train.py): rmsnorm closed forms (constant rows, gamma scaling) and a
 * float64 restatement; rmsnorm backward by finite differences; RoPE norm preservation,
 * backward(forward(x)) = x, position 0 identity and the 2x2 rotation by hand; embedding
 * backward as the transpose of the gather (<dW, W> = <dY, gather(W)>); cross entropy of equal
 * logits = log(vocab), gradient rows summing to 0, finite differences; Lion sign cases by hand. */
void ref_rmsnorm_forward(const float *x, const float *gamma, float *y, int64_t rows, int64_t dim, float eps);
void ref_rmsnorm_backward(const float *dy, const float *x, const float *gamma, float *dx, float *dgamma,
                          int64_t rows, int64_t dim, float eps);
void ref_rope(float *x, int64_t batch, int64_t seq, int64_t heads, int64_t head_dim, int64_t row_stride,
              float base, int64_t offset, int backward);
void ref_embedding_forward(const float *table, const uint32_t *ids, float *out, int64_t n, int64_t dim);
void ref_embedding_backward(const float *dy, const uint32_t *ids, float *dw, int64_t n, int64_t dim, int64_t vocab);
float ref_cross_entropy(const float *logits, const uint32_t *targets, float *losses, float *grad, int64_t rows,
                        int64_t vocab);
void ref_lion(float *w, float *m, const float *g, int64_t n, float lr, float beta1, float beta2, float wd,
              float scale);
double ref_sum_squares(const float *x, int64_t n);
float ref_fused_linear_cross_entropy(const float *hidden, const float *weight, const int32_t *targets, float *losses,
                                     float *grad_hidden, float *grad_weight, int64_t rows, int64_t hidden_dim,
                                     int64_t vocab);
void ref_fused_rmsnorm_linear(const float *x, const float *gamma, const float *w, float *out, int64_t rows,
                              int64_t hidden, int64_t out_features, float eps);

/* transpose_3d_f32 (src/shaders/attention.metal:163-182, called by transpose_3d_gpu,
 * src/ops/attention.rs:395-449): out[b][j][i] = in[b][i][j], in [batch][m][n].
 * Pinned by: numpy swapaxes on random data, involution (two transposes give the input back). */
void ref_transpose_3d(const float *in, float *out, int64_t batch, int64_t m, int64_t n);

/* causal_mask_3d_f32 (src/shaders/attention.metal:186-207, called by causal_mask_3d_gpu,
 * src/ops/attention.rs:455-517): out = col > row ? -inf : in over [batch][seq][seq].
 * Pinned by: numpy triu mask; the softmax of a masked constant row is 1/(row+1) on the
 * allowed columns (the causal prefix mean); a planted off-by-one (col >= row) is rejected. */
void ref_causal_mask_3d(const float *in, float *out, int64_t batch, int64_t seq);

#ifdef __cplusplus
}
#endif
#endif
