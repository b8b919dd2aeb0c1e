// Decode-shaped BF16 GEMM (M <= 16 rows): Y = alpha * X . W^T (+ beta * Y) (+ bias), X [M, K],
// W [N, K] row-major (the NT / Linear layout), FP32 accumulation. Same contract as it_gemm for these
// shapes (src/ops/bf16_ops/gemm.rs:25-146 with the transposed-operand form of
// src/ops/mps_gemm.rs:213-314); the greedy-decode shapes of the benchmark (M in {1, 4, 16},
// K 4096, N 11008) are HBM-bound: every W element is read once and used M times.
//
// Design: a 256-thread block owns 16 output columns (rows of W) and splits K over its 4 waves.
// Each wave streams its share of those W rows from HBM and feeds them to
// v_mfma_f32_16x16x32_bf16 as the B operand, with X (tiny, cache-resident) as the A operand.
//
// The operand layout wants lane l to hold row l%16, 8 consecutive k at 8*(l/16). Loaded that way,
// consecutive lanes read different rows, and the loads run at the speed of the lanes' addresses,
// not of the lines they touch: measured 28.3 us at M = 16 (K 4096, N 11008), against 20.4 us for the
// same loads issued with consecutive lanes on consecutive 16-byte chunks. So the loads come in pairs
// over a 64-wide k block, lane l reading row l/8 (first load) or 8 + l/8 (second), chunk l%8: each
// instruction reads 8 whole 128-byte lines, 8 consecutive lanes per line. Each pair goes through a
// 4 KB LDS slot of the wave (XOR-swizzled, no bank conflicts) into the operand layout of k 0-31 and
// 32-63 of the block; the wave's LDS accesses complete in order, so no barrier is needed. The loads
// are buffer loads whose range check zero-fills rows past N or M and chunks past the wave's k
// range, all issued before the first use (16 per lane and iteration at M > 8, 12 otherwise). The
// four partial tiles are summed through LDS in wave order and the epilogue writes the M valid rows.
// Measured at K 4096, N 11008 with cold weights: 18.7 / 19.8 / 20.6 us at M = 1 / 4 / 16 (the direct
// layout: 20.6 / 22.0 / 28.3 us). Two or four column blocks per wave sharing the X fragments
// measured slower: half or a quarter of the blocks.
#include <algorithm>

#include "epilogue.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int GV_THREADS = 256;
constexpr int GV_UNROLL = 8;   // 32-wide k chunks per wave per iteration (4 pairs of loads)
constexpr int GV_KCHUNK = 32;

// Weights are streamed once per call. The [K, N] kernel loads them nontemporally (measured 4-8%
// faster with cold weights); the [N, K] kernel measured 2-4% slower that way and loads them plainly.
__device__ __forceinline__ u32x4 wload_stream(const u32x4 *ptr) { return __builtin_nontemporal_load(ptr); }

__device__ __forceinline__ float out_load(const void *C, int64_t idx, bool bf16) {
    return bf16 ? bf16_to_f32(((const uint16_t *)C)[idx]) : ((const float *)C)[idx];
}

// Byte offset that a buffer load's range check turns into zeros without touching memory.
constexpr uint32_t GV_OOB = 0x80000000u;

// LDS slot (in 16-byte units) of row rr (0-7) and k chunk c (0-7) of one 8-row half of a pair:
// each row's 8 chunks fill 128 bytes, XOR-swizzled by the row so that 8 lanes reading one chunk
// of 8 rows hit 8 different bank groups.
__device__ __forceinline__ int gv_slot(int rr, int c) { return rr * 8 + (c ^ rr); }

// XHI: M > 8, so X rows 8-15 are loaded too (otherwise MFMA rows 8-15 of X repeat rows 0-7; they
// only reach output rows past M, which are not written).
template <bool XHI>
__global__ __launch_bounds__(GV_THREADS) void gemv_bf16_nt(const GemmArgs p) {
    // Per wave: two slots (pairs alternate), each W rows 0-7, W rows 8-15, X rows 0-7, X rows 8-15.
    __shared__ u32x4 stage[4][2][4][64];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int r = lane & 15, g = lane >> 4;   // operand layout: row r, k group g
    const int rl = lane >> 3, kc = lane & 7;  // load layout: row rl (+8), k chunk kc
    const int64_t n0 = (int64_t)blockIdx.x * 16;
    const int64_t z = blockIdx.y;
    const int64_t bo = z / p.batch_inner, bi = z % p.batch_inner;
    const uint16_t *X = (const uint16_t *)p.A + bo * p.sA_out + bi * p.sA_in;
    const uint16_t *W = (const uint16_t *)p.B + bo * p.sB_out + bi * p.sB_in + n0 * p.ldb;
    const int64_t coff = bo * p.sC_out + bi * p.sC_in;

    // Buffer descriptors over exactly the block's W rows and X's M rows (byte extents below 2^31,
    // checked by the host): rows past N or M, and chunks past the wave's k range (offset GV_OOB),
    // read as zeros with no memory access.
    const int64_t nrows = min((int64_t)16, p.N - n0);
    const __amdgpu_buffer_rsrc_t wrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(W), (short)0, (int)(((nrows - 1) * p.ldb + p.K) * 2), 0x00020000);
    const __amdgpu_buffer_rsrc_t xrs = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t *>(X), (short)0, (int)(((p.M - 1) * p.lda + p.K) * 2), 0x00020000);
    const uint32_t wo0 = (uint32_t)(rl * p.ldb * 2), wo1 = (uint32_t)((8 + rl) * p.ldb * 2);
    const uint32_t xo0 = (uint32_t)(rl * p.lda * 2), xo1 = (uint32_t)((8 + rl) * p.lda * 2);
    // LDS slots: where this lane's loaded chunk goes, and where its operand chunks come from.
    const int wslot = gv_slot(rl, kc);
    const int rq = r >> 3, rr = r & 7;
    const int lo_slot = gv_slot(rr, g), hi_slot = gv_slot(rr, 4 + g);
    const int xq = XHI ? rq : 0;

    // K split over the 4 waves in multiples of the 32-wide chunk.
    const int64_t span = ((p.K + 4 * GV_KCHUNK - 1) / (4 * GV_KCHUNK)) * GV_KCHUNK;
    const int64_t kb = wave * span, ke = min(p.K, kb + span);

    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int64_t k = kb; k < ke; k += GV_UNROLL * GV_KCHUNK) {
        u32x4 wr[GV_UNROLL], xr[GV_UNROLL];
#pragma unroll
        for (int pr = 0; pr < GV_UNROLL / 2; ++pr) {
            // This lane's chunk: 8 elements, and K % 8 == 0, so a chunk is whole or past the end.
            const int64_t kk = k + 64 * pr + 8 * kc;
            const bool ok = kk < ke;
            const uint32_t ko = (uint32_t)(kk * 2);
            wr[2 * pr] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? wo0 + ko : GV_OOB, 0, 0));
            wr[2 * pr + 1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(wrs, ok ? wo1 + ko : GV_OOB, 0, 0));
            xr[2 * pr] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, ok ? xo0 + ko : GV_OOB, 0, 0));
            if constexpr (XHI)
                xr[2 * pr + 1] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(xrs, ok ? xo1 + ko : GV_OOB, 0, 0));
        }
        // Every load is issued before the first use: left to itself the scheduler interleaves
        // them with the waits and keeps only a few in flight.
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int pr = 0; pr < GV_UNROLL / 2; ++pr) {
            // Through LDS from the load layout (lane: row rl, chunk kc) to the operand layout
            // (lane: row r, chunk g and 4 + g). A wave's LDS accesses complete in issue order, so
            // the slot written two pairs ago has been read, and the reads see these writes.
            u32x4 (&st)[4][64] = stage[wave][pr & 1];
            st[0][wslot] = wr[2 * pr];
            st[1][wslot] = wr[2 * pr + 1];
            st[2][wslot] = xr[2 * pr];
            if constexpr (XHI) st[3][wslot] = xr[2 * pr + 1];
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            const u32x4 wlo = st[rq][lo_slot], whi = st[rq][hi_slot];
            const u32x4 xlo = st[2 + xq][lo_slot], xhi = st[2 + xq][hi_slot];
            mma16<uint16_t>(acc, xlo, wlo);
            mma16<uint16_t>(acc, xhi, whi);
        }
    }
    // acc: lane l holds column n0 + l%16 and rows 4*(l/16) + i.
    // The four partial tiles go through each wave's own first slot (its reads of it are done).
    stage[wave][0][0][lane] = __builtin_bit_cast(u32x4, acc);
    __syncthreads();
    // Wave 0 sums the four K quarters in wave order and writes the tile.
    if (wave == 0) {
        f32x4 sum = __builtin_bit_cast(f32x4, stage[0][0][0][lane]);
#pragma unroll
        for (int w = 1; w < 4; ++w) sum += __builtin_bit_cast(f32x4, stage[w][0][0][lane]);
        const int64_t col = n0 + r;
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

// The buffer descriptors span 16 rows of W and M rows of X: byte extents and offsets below 2^31.
bool gemv_applicable(const GemmArgs &a, bool bf16, bool transA, bool transB) {
    return bf16 && !transA && transB && a.M >= 1 && a.M <= 16 && !a.dual && a.causal == CAUSAL_NONE &&
           a.kmode == KMODE_FULL && a.K % 8 == 0 && a.a_vec_ok && a.b_vec_ok && a.lda >= a.K &&
           a.ldb >= a.K && 16 * a.lda + a.K < (1ll << 30) && 16 * a.ldb + a.K < (1ll << 30) &&
           (a.N + 15) / 16 <= 0x7fffffff && a.batch <= 65535;
}

it_status launch_gemv(hipStream_t s, const GemmArgs &a) {
    dim3 grid((unsigned)((a.N + 15) / 16), (unsigned)a.batch);
    if (a.M > 8)
        hipLaunchKernelGGL(gemv_bf16_nt<true>, grid, dim3(GV_THREADS), 0, s, a);
    else
        hipLaunchKernelGGL(gemv_bf16_nt<false>, grid, dim3(GV_THREADS), 0, s, a);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
