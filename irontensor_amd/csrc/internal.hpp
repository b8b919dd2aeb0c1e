// Internal declarations shared by the runtime, the dispatch layer and the kernels.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <map>
#include <mutex>
#include <set>
#include <string>
#include <vector>

#include "irontensor_hip.h"

namespace it {

// ------------------------------------------------------------------ errors

// Records `msg` as this thread's last error and returns `st`.
it_status fail(it_status st, const std::string &msg);
it_status fail_hip(hipError_t err, const char *what);
void clear_error();

#define IT_HIP_TRY(expr)                                         \
    do {                                                         \
        hipError_t _e = (expr);                                  \
        if (_e != hipSuccess) return ::it::fail_hip(_e, #expr);  \
    } while (0)

// ------------------------------------------------------------------ context

struct ProfileRecord {
    std::string key;
    hipEvent_t start, stop;
};

struct ProfileStat {
    int64_t calls = 0;
    double total_ms = 0.0;
};

}  // namespace it

struct it_context {
    int device = 0;
    int num_cus = 0;
    int clock_khz = 0;
    char name[256] = {0};
    // Launches go to `stream`: the main stream, or the side stream between it_side_begin and
    // it_side_end (independent work, e.g. weight gradients, overlapping the main chain).
    hipStream_t stream = nullptr;
    hipStream_t main_stream = nullptr, side_stream = nullptr;
    int cur = 0;                 // 0 = main, 1 = side
    bool side_pending = false;   // side work not yet joined into the main stream
    hipEvent_t fork_ev = nullptr, join_ev = nullptr;

    // Caching allocator: freed blocks are kept per exact size and reused. Reuse is ordered on the
    // main stream; a free while side work is pending first makes the main stream wait for it.
    std::map<void *, size_t> live;
    std::multimap<size_t, void *> cache;
    size_t bytes_live = 0;

    // Library-owned scratch (split-K partials; attention recompute buffers), grown on demand, one
    // set per stream so concurrent main and side launches never share it.
    void *scratch[2] = {nullptr, nullptr};
    size_t scratch_bytes[2] = {0, 0};
    void *attn_scratch[2] = {nullptr, nullptr};
    size_t attn_scratch_bytes[2] = {0, 0};
    // Scratch blocks replaced by a larger one while graphs captured on this context were alive: a
    // graph keeps the addresses it was captured with, so the old block stays allocated until the
    // last such graph is destroyed (or the context shuts down).
    std::vector<std::pair<void *, size_t>> retired;
    std::set<it_graph *> graphs;  // graphs captured here and not yet destroyed
    // Arrival counters of kernels whose last block finishes a shared output (the decode kernel's
    // k splits), zeroed once at allocation; every launch leaves them zero.
    int *counters[2] = {nullptr, nullptr};

    // RoPE (cos, sin) tables per (seq, head_dim, base bits, position offset), built on first use
    // and kept until shutdown (every layer's forward and backward share one).
    std::map<std::vector<int64_t>, void *> rope_tables;

    // True between it_capture_begin and it_capture_end: nothing may allocate.
    bool capturing = false;

    // Profiler state.
    bool profiling = false;
    std::vector<it::ProfileRecord> pending;
    std::vector<hipEvent_t> event_pool;
    std::map<std::string, it::ProfileStat> stats;
};

struct it_event {
    hipEvent_t ev = nullptr;
};

struct it_graph {
    hipGraph_t graph = nullptr;
    hipGraphExec_t exec = nullptr;
    it_context *ctx = nullptr;  // the capturing context; NULL once it has shut down
};

namespace it {

// Waits for both streams.
it_status sync_all(it_context *ctx);
// Makes the main stream wait for the side stream's pending work.
it_status join_side(it_context *ctx);

// Grows the current stream's scratch to at least `bytes` (synchronises before freeing the old block).
it_status ensure_scratch(it_context *ctx, size_t bytes, void **out);
it_status ensure_attn_scratch(it_context *ctx, size_t bytes, void **out);
// The current stream's arrival counters (COUNTERS ints, zero), allocated on first use.
constexpr int64_t COUNTERS = 1 << 16;
it_status ensure_counters(it_context *ctx, int **out);

// Profiler hooks around one kernel launch.
void profile_begin(it_context *ctx, const std::string &key, hipEvent_t *start_out);
void profile_end(it_context *ctx, const std::string &key, hipEvent_t start);

// ------------------------------------------------------------------ kernel launch parameters

enum KMode : int {
    KMODE_FULL = 0,   // k in [0, K)
    KMODE_LOWER = 1,  // op(A)[m,k] == 0 for k > m: k in [0, min(K, m_block_end))
    KMODE_UPPER = 2,  // op(A)[m,k] == 0 for k < m: k in [m_block_begin, K)
};

enum CausalMode : int {
    CAUSAL_NONE = 0,
    CAUSAL_WRITE = 1,  // masked elements are written as -inf (the public epilogue)
    CAUSAL_SKIP = 2,   // fully masked tiles are not written (consumer is causal-aware)
};

struct GemmArgs {
    const void *A;
    const void *B;
    const void *B2;
    void *C;
    void *G;  // SwiGLU gate pre-activation (optional)
    void *U;  // SwiGLU up pre-activation (optional)
    const float *bias;
    float *partial;  // split-K partial sums [splits][batch][M][N] (f32)
    // Fused RMSNorm in front of the GEMM (FP32, A not transposed, one k split): op(A)[m,k] is
    // multiplied by a_kscale[k] on its way into LDS, the kernel sums the squares of each A row as
    // the tiles stream through, and the epilogue scales row m by 1 / sqrt(sum / K + rms_eps).
    // row_scale (optional, any GEMM): result row m multiplied by row_scale[m].
    const float *a_kscale;
    const float *row_scale;
    float rms_eps;
    int no_split;  // the planner must not split K
    // RoPE on the result (epilogue, 4-column vectors): columns < rope_cols rotate pairwise (2i,
    // 2i+1 of each head of 2 rope_half columns) by rope_table[(row % rope_seq) * rope_half + i].
    const float2 *rope_table;
    int64_t rope_seq, rope_cols;
    int rope_half;
    // SwiGLU backward (epilogue): the product is dL/dh; with the forward's gate G and up U ([M, N],
    // ld N) it writes dgate to C[row, col] and dup to C[row, N + col].
    int swiglu_bwd;
    // Softmax cross-entropy gradient in place of A (FP32, B not transposed): A holds logits
    // [tokens, classes]; op(A) rows are tokens (A not transposed) or k is the token (transposed).
    // Element x of token t, class c enters the product as
    // (exp(x - xent_stats[t].x) * xent_stats[t].y - (c == xent_tgt[t])) * xent_scale.
    const float2 *xent_stats;
    const uint32_t *xent_tgt;
    float xent_scale;

    int64_t M, N, K;
    int64_t lda, ldb, ldc;
    // Batch index z splits into (z / batch_inner, z % batch_inner) with separate strides.
    int64_t sA_in, sA_out, sB_in, sB_out, sC_in, sC_out;
    int64_t batch_inner;
    int64_t batch;
    int splits;
    int64_t k_per_split;  // multiple of the kernel's BK

    float alpha, beta;
    int has_bias;
    int dual;
    int causal;  // CausalMode
    int64_t causal_offset;
    int kmode;  // KMode
    int out_bf16;
    int a_vec_ok, b_vec_ok;  // 16-byte vector loads are legal for the operand
    int c_vec_ok;            // 4-element vector loads/stores of C (and G, U) are legal
    int tiles_m, tiles_n;
};

// Launches the MFMA GEMM for `dtype_in` (IT_F32 / IT_BF16). Chooses tile shape and split-K.
it_status launch_gemm(it_context *ctx, it_dtype dtype_in, bool transA, bool transB, GemmArgs args,
                      const char *profile_tag);
// `count` (<= 8) independent GEMMs of one dtype (ta[i], tb[i]: their layouts): grouped launches
// where they pay (kernels_gemm.hip), else launch_gemm for each.
it_status launch_gemm_group(it_context *ctx, it_dtype dtype_in, const bool *ta, const bool *tb, GemmArgs *args,
                            int count, const char *profile_tag);

// Fused attention (kernels_flash.hip), head_dim 64. Per-head addressing of each operand:
// (bh / heads) * bs + (bh % heads) * hs + row * rs + col (element strides).
struct FlashArgs {
    const void *Q, *K, *V, *dO;  // operand dtype
    void *O;                     // forward output / backward input (f32, or BF16 with o_bf16)
    float *lse, *dlt;            // [bh][sq] row log-sum-exp; dlt: workspace of 2 [bh][sq] row arrays
                                 // (FP32 kernels: rowsum(dO * O) in the first; BF16 kernels:
                                 // -rowsum(dO * O), then -LSE log2 e)
    void *dQ, *dK, *dV;          // gradients (f32, or BF16 with grad_bf16)
    int o_bf16, grad_bf16;       // BF16 O / gradients (RNE): the BF16 (flash2) kernels only
    int64_t bh, sq, skv, head_dim, heads;
    int64_t q_bs, q_hs, q_rs;     // Q and dQ
    int64_t kv_bs, kv_hs, kv_rs;  // K, V, dK, dV
    int64_t o_bs, o_hs, o_rs;     // O
    int64_t do_bs, do_hs, do_rs;  // dO
    float scale;
    int causal;
};
// Decode-shaped BF16 NT GEMM (M <= 16), HBM-bound: kernels_gemv.hip.
bool gemv_applicable(const GemmArgs &a, bool bf16, bool transA, bool transB);
it_status launch_gemv(hipStream_t s, const GemmArgs &a);
// Decode-shaped BF16 GEMM with the weight stored [K, N] (NN, and TN with X stored [K, M]), M <= 16:
// gemv_kn_splits picks the k splits; with more than one, a.partial must hold
// splits * batch * M * N floats and `counters` one zero int per (column strip, batch item).
bool gemv_kn_applicable(const GemmArgs &a, bool bf16, bool transA, bool transB);
int gemv_kn_splits(const GemmArgs &a, bool transA);
int gemv_kn_min_splits(const GemmArgs &a, bool transA);
int64_t gemv_kn_strips(const GemmArgs &a);
it_status launch_gemv_kn(hipStream_t s, bool transA, const GemmArgs &a, int *counters);

bool flash_supported(const FlashArgs &p, int elem_bytes, bool backward);
// BF16 forms on 32x32x16 MFMAs with direct-to-LDS tile loads (kernels_flash2.hip); the launchers of
// kernels_flash.hip hand BF16 work to them when flash2_applicable.
bool flash2_applicable(const FlashArgs &p, bool backward);
it_status launch_flash2_fwd(hipStream_t s, const FlashArgs &p);
it_status launch_flash2_bwd(hipStream_t s, const FlashArgs &p);
// The static device workspace of the no-allocation entry points (noalloc.hip): noalloc_init looks
// up this device's copy (called by it_init with the device current); noalloc_scratch returns its
// device address, or NULL before that.
it_status noalloc_init(int device);
void *noalloc_scratch(int device);
it_status launch_flash_fwd(hipStream_t s, const FlashArgs &p, bool bf16);
it_status launch_flash_bwd(hipStream_t s, const FlashArgs &p, bool bf16);

// Elementwise and row kernels (kernels_misc.hip).
it_status launch_zero(hipStream_t s, void *dst, size_t bytes);
it_status launch_f32_to_bf16(hipStream_t s, const float *src, uint16_t *dst, int64_t n);
it_status launch_bf16_to_f32(hipStream_t s, const uint16_t *src, float *dst, int64_t n);
it_status launch_softmax_rows(hipStream_t s, const float *S, void *P, int p_bf16, int64_t batch,
                              int64_t rows, int64_t cols, int causal, int64_t causal_offset,
                              int64_t s_ld_batch, int64_t p_ld_batch);
it_status launch_softmax_backward(hipStream_t s, const float *dY, const void *Y, int y_bf16,
                                  void *dX, int dx_bf16, int64_t batch, int64_t rows,
                                  int64_t cols, int causal);
it_status launch_splitk_reduce(hipStream_t s, const GemmArgs &a);
it_status launch_transpose_3d(hipStream_t s, const float *in, float *out, int64_t batch, int64_t m, int64_t n);
it_status launch_causal_mask_3d(hipStream_t s, const float *in, float *out, int64_t batch, int64_t seq);
it_status launch_fill_normal(hipStream_t s, bool bf16, void *dst, uint64_t seed, int64_t offset, int64_t n,
                             double std_dev);

// Training-step ops around the contractions (kernels_train.hip).
it_status launch_rmsnorm_forward(hipStream_t s, bool y_bf16, int64_t rows, int64_t dim, float eps, const float *x,
                                 const float *res, const float *gamma, float *sum_out, void *y);
int64_t rmsnorm_backward_scratch_bytes(int64_t rows, int64_t dim);
it_status launch_rmsnorm_backward(hipStream_t s, int64_t rows, int64_t dim, float eps, const float *dy,
                                  const float *x, const float *gamma, const float *gres, float *dx,
                                  float *dgamma, float *part);
it_status launch_rope_table(hipStream_t s, int64_t seq, int64_t head_dim, float base, int64_t offset, void *table);
// The context's (cos, sin) table for these parameters, built on first use (not during capture).
it_status rope_table(it_context *ctx, int64_t seq, int64_t head_dim, float base, int64_t offset, const void **out);
it_status launch_rope(hipStream_t s, bool src_bf16, bool dst_bf16, int64_t batch, int64_t seq, int64_t heads,
                      int64_t head_dim, const void *table, int backward, const void *src, int64_t src_rs,
                      void *dst, int64_t dst_rs, int64_t copy_cols);
it_status launch_embedding_forward(hipStream_t s, bool table_bf16, bool out_bf16, int64_t n, int64_t dim,
                                   int64_t vocab, const void *table, const uint32_t *ids, void *out);
it_status launch_embedding_backward(hipStream_t s, int64_t n, int64_t dim, int64_t vocab, const float *dy,
                                    const uint32_t *ids, float *dw);
it_status launch_cross_entropy(hipStream_t s, bool grad_bf16, int64_t rows, int64_t vocab, const float *logits,
                               const uint32_t *targets, float *losses, void *grad, float *stats, float *loss_mean,
                               bool vec_ok);
it_status launch_swiglu_backward(hipStream_t s, bool in_bf16, bool out_bf16, int64_t rows, int64_t cols,
                                 const float *dh, int64_t ld_dh, const void *gate, const void *up, int64_t ld_gu,
                                 void *dgate, void *dup, int64_t ld_out);
it_status launch_flce_chunk_stats(hipStream_t s, const float *x, int64_t ld, int64_t rows, int64_t vc, int64_t v0,
                                  const int32_t *targets, int64_t vocab, void *stats, int64_t nchunks, int64_t chunk,
                                  float *tlogit);
it_status launch_flce_combine(hipStream_t s, const void *stats, int64_t nchunks, const float *tlogit,
                              const int32_t *targets, int64_t vocab, int64_t rows, float *lse, float *losses,
                              float *mean_out, float *scale_out);
it_status launch_flce_chunk_grad(hipStream_t s, float *x, int64_t ld, int64_t rows, int64_t vc, int64_t v0,
                                 const int32_t *targets, int64_t vocab, const float *lse);
it_status launch_scale_by_device(hipStream_t s, float *x, int64_t n, const float *scale);
int64_t grad_norm_partials(int count, const int64_t *n);
it_status launch_grad_norm(hipStream_t s, int count, const float *const *g, const int64_t *n, float max_norm,
                           float *out, double *part);
it_status launch_lion(hipStream_t s, int count, float *const *w, float *const *m, const float *const *g,
                      const int64_t *n, float lr, float beta1, float beta2, float wd, const float *scale_dev,
                      const float *lr_dev);

}  // namespace it
