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
#include <algorithm>

#include "epilogue.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int GV_THREADS = 256;
constexpr int GV_UNROLL = 8;   // 32-wide k chunks per wave per iteration
constexpr int GV_KCHUNK = 32;
constexpr int GV_NB = 1;       // 16-column blocks per wave (they would share the X fragments)

// Weights are streamed once per call. The [K, N] kernel loads them nontemporally (measured 4-8%
// faster with cold weights); the [N, K] kernel measured 2-4% slower that way and loads them plainly.
__device__ __forceinline__ u32x4 wload_stream(const u32x4 *ptr) { return __builtin_nontemporal_load(ptr); }

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

// Decode-shaped BF16 GEMM with the weight stored [K, N] (the NN layout Y = X.W, and TN, Y = X^T.W
// with X stored [K, M]): same contract as it_gemm (src/ops/bf16_ops/gemm.rs:25-146 with the
// operand forms of src/ops/mps_gemm.rs:44-202,325-426). HBM-bound like the NT form: each W element
// is read once and used M times.
//
// W's k-rows are N-contiguous, while an MFMA operand lane needs 8 consecutive k of one column.
// Lane (g = l / 16, c = l % 16) of a wave therefore loads an 8 x 8 block of W, rows k .. k + 7 of
// its k-chunk group g and columns 8c .. 8c + 7 of the block's 128-column strip (each load
// instruction: 16 lanes x 16 bytes = 256 contiguous bytes of one k-row), and transposes it in
// registers with v_perm_b32 (4 per column). Column j of the block then feeds MFMA j as the B
// operand (lane c: column 8c + j), so the 8 MFMAs of a 32-wide k chunk cover the strip's 128
// columns, X (rows l % 16 < M, the tiny cache-resident operand) being the A operand; a lane ends
// with 8 consecutive output columns of rows 4g .. 4g + 3. K is split over the 4 waves (summed in
// LDS in wave order) and, for enough blocks in flight, over blockIdx.y splits whose partial sums
// go through the ordered split-K reduction.
constexpr int GK_STRIP = 128;  // output columns per block
#ifndef GK_WAVES
#define GK_WAVES 4  // waves per block (k split among them)
#endif
#ifndef GK_UNROLL
#define GK_UNROLL 2  // 32-wide k chunks per wave per iteration
#endif
constexpr int GK_THREADS = 64 * GK_WAVES;
constexpr int GV_DEVICE_SCOPE = 16;  // cache-policy bit sc1 of the buffer intrinsics: device scope
constexpr int GK_XT_BYTES = 32768;   // LDS for the transposed X slice of the TN form

template <bool TA>
__global__ __launch_bounds__(GK_THREADS) void gemv_bf16_kn(const GemmArgs p, int *counters) {
    __shared__ f32x4 part[GK_WAVES - 1][8][64];
    __shared__ __attribute__((aligned(16))) uint16_t xt[TA ? GK_XT_BYTES / 2 : 8];  // [M][k range]
    __shared__ int last;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int c = lane & 15, g = lane >> 4;
    const int64_t n0 = (int64_t)blockIdx.x * GK_STRIP + 8 * c;  // this lane's 8 columns
    const int64_t z = blockIdx.y;
    const int64_t b = z % p.batch, split = z / p.batch;
    const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
    const uint16_t *X = (const uint16_t *)p.A + bo * p.sA_out + bi * p.sA_in;
    const uint16_t *W = (const uint16_t *)p.B + bo * p.sB_out + bi * p.sB_in;
    const int64_t coff = bo * p.sC_out + bi * p.sC_in;
    // The split's k range, and this wave's part of it in whole 32-wide chunks (K % 32 == 0).
    const int64_t kb = split * p.k_per_split, ke = min(p.K, kb + p.k_per_split);
    const int64_t span = ((ke - kb + 32 * GK_WAVES - 1) / (32 * GK_WAVES)) * 32;
    const int64_t kw0 = min(ke, kb + wave * span), kw1 = min(ke, kw0 + span);
    const bool col_ok = n0 < p.N;  // N % 8 == 0: a lane's 8 columns are all in range or all out
    const bool row_ok = c < p.M;
    const uint16_t *wcol = W + (col_ok ? n0 : 0);
    const int64_t kr = ke - kb;
    if constexpr (TA) {
        // X stored [K, M]: its k rows of this split, transposed into LDS as [M][kr] so a lane's
        // 8 consecutive k are one 16-byte read (kr * M * 2 <= GK_XT_BYTES, checked by the host).
        // Contiguous rows (lda == M, a power of two) and an aligned base: 16-byte loads.
        const int M = (int)p.M, krr = (int)kr;
        const uint16_t *src = X + kb * p.lda;
        if (p.lda == p.M && (M & (M - 1)) == 0 && ((uintptr_t)src & 15) == 0) {
            const int msh = __builtin_ctz(M);
            for (int ch = tid; ch < (krr << msh) / 8; ch += GK_THREADS) {
                const u32x4 v = *(const u32x4 *)(src + ch * 8);
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    const int el = ch * 8 + e;
                    xt[(el & (M - 1)) * krr + (el >> msh)] = (uint16_t)(v[e >> 1] >> (16 * (e & 1)));
                }
            }
        } else {
            for (int e = tid; e < krr * M; e += GK_THREADS) {
                const int kk = e / M, m = e - kk * M;
                xt[m * krr + kk] = src[kk * p.lda + m];
            }
        }
        __syncthreads();
    }

    f32x4 acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
    for (int64_t k = kw0; k < kw1; k += 32 * GK_UNROLL) {
        u32x4 w[GK_UNROLL][8], x[GK_UNROLL];
#pragma unroll
        for (int u = 0; u < GK_UNROLL; ++u) {
            const bool ok = k + 32 * u < kw1;
            const int64_t kk = (ok ? k + 32 * u : kw0) + 8 * g;  // first k-row of this lane's block
#pragma unroll
            for (int r = 0; r < 8; ++r) {
                const u32x4 v = wload_stream((const u32x4 *)(wcol + (kk + r) * p.ldb));
                w[u][r] = ok && col_ok ? v : u32x4{0u, 0u, 0u, 0u};
            }
            x[u] = u32x4{0u, 0u, 0u, 0u};
            if (ok && row_ok) {
                if constexpr (TA)
                    x[u] = *(const u32x4 *)(xt + c * kr + (kk - kb));
                else
                    x[u] = *(const u32x4 *)(X + c * p.lda + kk);
            }
        }
#pragma unroll
        for (int u = 0; u < GK_UNROLL; ++u)
#pragma unroll
            for (int j = 0; j < 8; ++j) {
                // column j of the 8 x 8 block, k-pairs packed low/high as the MFMA operand wants
                const uint32_t sel = (j & 1) ? 0x07060302u : 0x05040100u;
                u32x4 f;
#pragma unroll
                for (int e = 0; e < 4; ++e)
                    f[e] = __builtin_amdgcn_perm(w[u][2 * e + 1][j >> 1], w[u][2 * e][j >> 1], sel);
                mma16<uint16_t>(acc[j], x[u], f);
            }
    }
    if (wave > 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) part[wave - 1][j][lane] = acc[j];
    }
    __syncthreads();
    // acc[j][i] of wave 0: row 4g + i, column n0 + j, summed over the waves in wave order.
    if (p.splits == 1) {
        if (wave != 0) return;
#pragma unroll
        for (int w2 = 0; w2 < GK_WAVES - 1; ++w2)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += part[w2][j][lane];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            finish4<true, true>(p, f32x4{acc[0][i], acc[1][i], acc[2][i], acc[3][i]}, 4 * g + i, n0, coff, 0);
            finish4<true, true>(p, f32x4{acc[4][i], acc[5][i], acc[6][i], acc[7][i]}, 4 * g + i, n0 + 4, coff, 0);
        }
        return;
    }
    // Partial sums [split][batch][M][N] at device scope (written through the XCD's L2); the
    // strip's last block to arrive adds all of them in split order and finishes the strip. Wave
    // w < 4 handles row 4g + w of each lane's four rows.
    const __amdgpu_buffer_rsrc_t prt =
        __builtin_amdgcn_make_buffer_rsrc(p.partial, (short)0, (int)(p.splits * p.batch * p.M * p.N * 4), 0x00020000);
    const int i = wave;
    const int64_t row = 4 * g + i;
    const bool mine = wave < 4 && col_ok && row < p.M;
    if (wave == 0) {
#pragma unroll
        for (int w2 = 0; w2 < GK_WAVES - 1; ++w2)
#pragma unroll
            for (int j = 0; j < 8; ++j) acc[j] += part[w2][j][lane];
    }
    __syncthreads();  // every wave has read its LDS partials
    if (wave == 0) {
#pragma unroll
        for (int j = 0; j < 8; ++j) part[0][j][lane] = acc[j];  // the block's sums, for waves 1-3
    }
    __syncthreads();
    if (mine) {
        f32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            lo[e] = part[0][e][lane][i];
            hi[e] = part[0][4 + e][lane][i];
        }
        const uint32_t off = (uint32_t)(((z * p.M + row) * p.N + n0) * 4);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, lo), prt, off, 0, GV_DEVICE_SCOPE);
        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, hi), prt, off + 16, 0, GV_DEVICE_SCOPE);
    }
    __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's partial has reached device scope
    __syncthreads();
    int *cnt = counters + blockIdx.x * p.batch + b;
    if (tid == 0) {
        // The hand-off is ordered by the hardware's scoped accesses, not by release/acquire: the
        // partials were stored at device scope (written through this XCD's L2) and the vmcnt(0)
        // wait above held the arrival back until those stores completed; the last block's
        // device-scope loads below are issued after its arrival returns (the barrier) and miss
        // its own L2. Release/acquire atomics at agent scope would write back and invalidate the
        // whole XCD L2 per block: measured 2.4x slower at M = 1 (NN 19.6 -> 47 us).
        const int old = __hip_atomic_fetch_add(cnt, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        last = old == p.splits - 1;
        if (last) __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    __syncthreads();
    if (!last || !mine) return;
    f32x4 lo = {0.f, 0.f, 0.f, 0.f}, hi = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 8
    for (int sp = 0; sp < p.splits; ++sp) {
        const uint32_t off = (uint32_t)((((sp * p.batch + b) * p.M + row) * p.N + n0) * 4);
        lo += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prt, off, 0, GV_DEVICE_SCOPE));
        hi += __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(prt, off + 16, 0, GV_DEVICE_SCOPE));
    }
    finish4<true, true>(p, lo, row, n0, coff, 0);
    finish4<true, true>(p, hi, row, n0 + 4, coff, 0);
}

}  // namespace

int64_t gemv_kn_strips(const GemmArgs &a) { return (a.N + GK_STRIP - 1) / GK_STRIP; }

// The fewest k splits the TN form's LDS slice of X allows.
int gemv_kn_min_splits(const GemmArgs &a, bool transA) {
    int64_t ks = 1;
    if (transA)
        while (((a.K + ks - 1) / ks + 127) / 128 * 128 * a.M * 2 > GK_XT_BYTES) ++ks;
    return (int)ks;
}

// Splits of K: about 2 blocks per column strip (172 blocks at N = 11008); NN with M <= 4 measured
// 3-8% faster with about 8 (688 blocks), TN and M = 16 slower.
int gemv_kn_splits(const GemmArgs &a, bool transA) {
    const int64_t strips = gemv_kn_strips(a);
    const int64_t target = !transA && a.M <= 4 ? 688 : 172;
    int64_t ks = std::max<int64_t>(1, (target + strips * a.batch - 1) / (strips * a.batch));
    ks = std::min<int64_t>({ks, std::max<int64_t>(1, a.K / 512), 32});
    while (ks > 1 && ks * a.batch > 65535) --ks;
    return (int)std::max<int64_t>(ks, gemv_kn_min_splits(a, transA));
}

// The partial sums are addressed with 32-bit byte offsets: splits * batch * M * N * 4 < 2^31 (the TN
// form may need more than 32 splits for its LDS slice of X).
bool gemv_kn_applicable(const GemmArgs &a, bool bf16, bool transA, bool transB) {
    return bf16 && !transB && a.M >= 1 && a.M <= 16 && !a.dual && a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL &&
           !a.swiglu_bwd && !a.xent_stats && !a.a_kscale && !a.rope_table && a.K % 32 == 0 && a.N % 8 == 0 &&
           a.ldb % 8 == 0 && a.b_vec_ok && (transA || (a.a_vec_ok && a.lda % 8 == 0)) &&
           gemv_kn_strips(a) * a.batch <= COUNTERS && a.batch * a.M * a.N <= (1ll << 24) &&
           (int64_t)gemv_kn_splits(a, transA) * a.batch * a.M * a.N * 4 < (1ll << 31);
}

it_status launch_gemv_kn(hipStream_t s, bool transA, const GemmArgs &a, int *counters) {
    dim3 grid((unsigned)gemv_kn_strips(a), (unsigned)(a.batch * a.splits));
    if (transA)
        hipLaunchKernelGGL(gemv_bf16_kn<true>, grid, dim3(GK_THREADS), 0, s, a, counters);
    else
        hipLaunchKernelGGL(gemv_bf16_kn<false>, grid, dim3(GK_THREADS), 0, s, a, counters);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

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
