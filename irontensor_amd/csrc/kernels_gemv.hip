// Decode-shaped BF16 GEMM (M <= 16 rows): Y = alpha * X . W^T (+ beta * Y) (+ bias), X [M, K],
// W [N, K] row-major (the NT / Linear layout), FP32 accumulation. Same contract as it_gemm for these
// shapes (src/ops/bf16_ops/gemm.rs:25-146 with the transposed-operand form of
// src/ops/mps_gemm.rs:213-314); the greedy-decode shapes of the benchmark (M in {1, 4, 16},
// K 4096, N 11008) are HBM-bound: every W element is read once and used M times.
//
// Design: a 256-thread block owns 16 * GV_NB output columns (rows of W) and splits K over its 4
// waves. Each wave streams its share of those W rows straight from HBM as the B operand of
// v_mfma_f32_16x16x32_bf16 (lane l: W row n0 + l%16, 8 consecutive k at 8*(l/16)), eight 16-byte
// loads in flight per lane and column block, with X (tiny, cache-resident) as the A operand (row
// l%16; lanes past M load nothing and feed zeros). No LDS staging: each W byte is loaded once, by
// the lane that feeds it to the MFMA. The four partial tiles are summed through LDS and the
// epilogue writes the M valid rows. One column block per wave measured fastest at M = 1 and 4
// (two blocks per wave halve the X requests but halve the number of blocks).
#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int GV_THREADS = 256;
constexpr int GV_UNROLL = 8;   // 32-wide k chunks per wave per iteration
constexpr int GV_KCHUNK = 32;
constexpr int GV_NB = 1;       // 16-column blocks per wave (they would share the X fragments)

__device__ __forceinline__ float out_load(const void *C, int64_t idx, bool bf16) {
    return bf16 ? bf16_to_f32(((const uint16_t *)C)[idx]) : ((const float *)C)[idx];
}

__global__ __launch_bounds__(GV_THREADS) void gemv_bf16_nt(const GemmArgs p) {
    __shared__ f32x4 part[4][GV_NB][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * (16 * GV_NB);
    const int64_t z = blockIdx.y;
    const int64_t bo = z / p.batch_inner, bi = z % p.batch_inner;
    const uint16_t *X = (const uint16_t *)p.A + bo * p.sA_out + bi * p.sA_in;
    const uint16_t *W = (const uint16_t *)p.B + bo * p.sB_out + bi * p.sB_in;
    const int64_t coff = bo * p.sC_out + bi * p.sC_in;

    // K split over the 4 waves in multiples of the 32-wide chunk.
    const int64_t span = ((p.K + 4 * GV_KCHUNK - 1) / (4 * GV_KCHUNK)) * GV_KCHUNK;
    const int64_t kb = wave * span, ke = min(p.K, kb + span);
    const bool xrow_ok = r < p.M;
    const uint16_t *xrow = X + (xrow_ok ? r * p.lda : 0) + 8 * g;
    const uint16_t *wrow[GV_NB];
    bool wrow_ok[GV_NB];
#pragma unroll
    for (int j = 0; j < GV_NB; ++j) {
        wrow_ok[j] = n0 + 16 * j + r < p.N;
        wrow[j] = W + (wrow_ok[j] ? (n0 + 16 * j + r) * p.ldb : 0) + 8 * g;
    }

    f32x4 acc[GV_NB];
#pragma unroll
    for (int j = 0; j < GV_NB; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int64_t k = kb; k < ke; k += GV_UNROLL * GV_KCHUNK) {
        u32x4 wf[GV_NB][GV_UNROLL], xf[GV_UNROLL];
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u) {
            const int64_t kk = k + u * GV_KCHUNK;
            // Chunks are 8 elements and K % 8 == 0, so a chunk is either whole or past the end.
            const bool ok = kk + 8 * g < ke;
#pragma unroll
            for (int j = 0; j < GV_NB; ++j) {
                const u32x4 w = *(const u32x4 *)(wrow[j] + (ok ? kk : kb));
                wf[j][u] = (ok && wrow_ok[j]) ? w : u32x4{0u, 0u, 0u, 0u};
            }
            // X rows past M are zero; their lanes issue no load.
            xf[u] = u32x4{0u, 0u, 0u, 0u};
            if (ok && xrow_ok) xf[u] = *(const u32x4 *)(xrow + kk);
        }
#pragma unroll
        for (int u = 0; u < GV_UNROLL; ++u)
#pragma unroll
            for (int j = 0; j < GV_NB; ++j) mma16<uint16_t>(acc[j], xf[u], wf[j][u]);
    }
    // acc[j]: lane l holds column n0 + 16j + l%16 and rows 4*(l/16) + i.
#pragma unroll
    for (int j = 0; j < GV_NB; ++j) part[wave][j][lane] = acc[j];
    __syncthreads();
    // Wave j (< GV_NB) sums column block j over the four K quarters and writes it.
    if (wave < GV_NB) {
        const int j = wave;
        f32x4 sum = part[0][j][lane];
#pragma unroll
        for (int w = 1; w < 4; ++w) sum += part[w][j][lane];
        const int64_t col = n0 + 16 * j + r;
        if (col < p.N) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int64_t row = 4 * g + i;
                if (row >= p.M) continue;
                const int64_t idx = coff + row * p.ldc + col;
                float v = p.alpha * sum[i];
                if (p.beta != 0.f) v += p.beta * out_load(p.C, idx, p.out_bf16);
                if (p.has_bias) v += p.bias[col];
                if (p.out_bf16)
                    ((uint16_t *)p.C)[idx] = f32_to_bf16_rne(v);
                else
                    ((float *)p.C)[idx] = v;
            }
        }
    }
}

}  // namespace

bool gemv_applicable(const GemmArgs &a, bool bf16, bool transA, bool transB) {
    return bf16 && !transA && transB && a.M >= 1 && a.M <= 16 && !a.dual && a.causal == CAUSAL_NONE &&
           a.kmode == KMODE_FULL && a.K % 8 == 0 && a.a_vec_ok && a.b_vec_ok &&
           (a.N + 15) / 16 <= 0x7fffffff && a.batch <= 65535;
}

it_status launch_gemv(hipStream_t s, const GemmArgs &a) {
    dim3 grid((unsigned)((a.N + 16 * GV_NB - 1) / (16 * GV_NB)), (unsigned)a.batch);
    hipLaunchKernelGGL(gemv_bf16_nt, grid, dim3(GV_THREADS), 0, s, a);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
