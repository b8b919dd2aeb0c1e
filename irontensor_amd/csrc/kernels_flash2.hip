// Fused attention for BF16 operands, head_dim 64, on v_mfma_f32_32x32x16_bf16: the same mathematics
// as kernels_flash.hip (ops::attention and attention_backward_recompute, src/ops/attention.rs:286-377,
// src/train/helpers.rs:120-193), laid out for fewer re-reads, no register transposes and a lean
// softmax:
//
//   * 128 rows (queries, or keys for dK/dV) per workgroup, 32 per wave, 64-row tiles of the other
//     side streamed through LDS, so each K/V (or Q/dO) tile is read from L2 once per 128 rows.
//   * Tiles move global -> LDS directly (buffer_load_dwordx4 ... lds), 64 rows x 128 bytes, the
//     16-byte chunk c of row r at position c ^ swz(r), swz(r) = 4 ((r >> 1) & 1) + ((r >> 2) & 3).
//     Fragments are read row-major (one ds_read_b128: 32 rows x 8 d) or transposed (two
//     ds_read_tr16_b64: 32 d-columns x 8 rows); with this swizzle both read patterns hit distinct
//     banks. Two stages in two LDS objects; the loads of tile t+2 go out after the barrier that ends
//     the reads of tile t.
//   * Products are oriented so that a lane's 32x32 accumulator holds one column (a query, or a key
//     in dK/dV) and 16 rows: S^T = K.Q^T in the forward and dQ kernels (row statistics: one
//     cross-lane shuffle), S = Q.K^T in the dK/dV kernel. Probabilities and dS feed the next MFMA
//     from the accumulators as B operands; the LDS operand they meet (V^T, K^T, dO^T, Q^T) is read
//     transposed with the same k order: lane group h = l / 32 holds rows 4h..4h+3 and 8+4h..8+4h+3
//     of each 16-row chunk.
//   * Forward softmax, per 32-key half tile: the row max is taken on the raw scores, probabilities
//     are exp2(s * scale * log2 e - m) (one FMA and one v_exp_f32 each), and the output and row sum
//     are rescaled only when the running max grows by more than 8 (log2 units: probabilities then
//     stay below 2^8 and the final division by the row sum cancels the factor); the row sum adds
//     the FP32 probabilities, and P is rounded to BF16 before its MFMA.
// The backward is deterministic (dQ and dK/dV from two kernels, no atomics). O (written by the
// forward, read by the backward's row pass) and dQ, dK, dV are FP32, or BF16 (round to nearest
// even) when the caller asks for BF16 outputs.
#include <cmath>

#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int HD = 64;      // head dim
constexpr int RB = 128;     // rows per workgroup
constexpr int TR = 64;      // rows per streamed tile
constexpr int TB = TR * 128;  // bytes per tile
constexpr int NTH = 256;
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;
constexpr float RESCALE = 8.f;  // lazy rescale threshold, log2 units

typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;
typedef __attribute__((address_space(3))) void lds_void_t;

__device__ __forceinline__ int swz(int r) { return (((r >> 1) & 1) << 2) | ((r >> 2) & 3); }

__device__ __forceinline__ f32x16 mfma32(const u32x4 &a, const u32x4 &b, const f32x16 &c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                   0, 0, 0);
}

__device__ __forceinline__ f32x16 zero16() {
    return f32x16{0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
}

// Fragment reads of a 64-row tile (128 bytes per row, swizzled as above):
//   row-major    lane l reads row r0 + l % 32, d = 16 ks + 8 (l / 32) .. +7 (one ds_read_b128);
//   transposed   lane l gets column c0 + l % 32 at tile rows k0 + 4h + 0..3 and k0 + 8 + 4h + 0..3
//                (h = l / 32), from two ds_read_tr16_b64: that instruction hands lane i of a 16-lane
//                group the 4 rows its group points at (lane j of the group points at row j / 4,
//                columns 4 (j % 4) .. +3).
// Per-lane LDS byte offsets of these reads are computed once per kernel: the swizzle depends only on
// row bits 1..3, so the row block (a multiple of 16 rows), the k chunk of a transposed read and the
// stage are compile-time offsets added to them (ds_read immediates). Kept opaque so the compiler
// holds them in 8 registers instead of hoisting a swizzled address per read out of the loop.
struct FragOff {
    uint32_t rm[4];     // row-major at r0 = 0, ks = 0..3
    uint32_t tr[2][2];  // transposed at c0 = 32 dh, k0 = 0: rows r1 (lo) and r1 + 8 (hi)
};

__device__ __forceinline__ FragOff frag_offsets(int lane) {
    FragOff f;
    const int r = lane & 31;
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) f.rm[ks] = (uint32_t)(r * 128 + (((2 * ks + (lane >> 5)) ^ swz(r)) << 4));
    const int g = lane >> 4, j = lane & 15;
    const int r1 = 4 * (g >> 1) + (j >> 2), r2 = r1 + 8, half = (j & 1) << 3;
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) {
        const int chunk = (32 * dh + 16 * (g & 1) + 4 * (j & 3)) >> 3;
        f.tr[dh][0] = (uint32_t)(r1 * 128 + ((chunk ^ swz(r1)) << 4) + half);
        f.tr[dh][1] = (uint32_t)(r2 * 128 + ((chunk ^ swz(r2)) << 4) + half);
    }
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) asm volatile("" : "+v"(f.rm[ks]));
#pragma unroll
    for (int dh = 0; dh < 2; ++dh) asm volatile("" : "+v"(f.tr[dh][0]), "+v"(f.tr[dh][1]));
    return f;
}

// Row-major fragment at row r0 (a multiple of 16), k step ks.
__device__ __forceinline__ u32x4 frag_rm_o(const char *tile, const FragOff &f, int r0, int ks) {
    return *(const u32x4 *)(tile + r0 * 128 + f.rm[ks]);
}

// Transposed fragment at column c0 (0 or 32), row k0 (a multiple of 16).
__device__ __forceinline__ u32x4 frag_tr_o(const char *tile, const FragOff &f, int c0, int k0) {
    const int dh = c0 >> 5;
    const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(tile + k0 * 128 + f.tr[dh][0]));
    const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(tile + k0 * 128 + f.tr[dh][1]));
    const u32x2 a = __builtin_bit_cast(u32x2, lo), b = __builtin_bit_cast(u32x2, hi);
    return u32x4{a[0], a[1], b[0], b[1]};
}

// B operand from accumulator values j0 .. j0 + 7 of a 32x32 block (a 16-row chunk), rounded to BF16.
__device__ __forceinline__ u32x4 pack8(const f32x16 &v, int j0) {
    return u32x4{pack_bf16x2(v[j0], v[j0 + 1]), pack_bf16x2(v[j0 + 2], v[j0 + 3]), pack_bf16x2(v[j0 + 4], v[j0 + 5]),
                 pack_bf16x2(v[j0 + 6], v[j0 + 7])};
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t rsrc(const void *base, int64_t bytes) {
    const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

// One operand streamed in 64-row tiles. Load instruction i (0, 1) of wave w fills rows 8 (2w + i)
// .. +7 of the tile: lane L takes row L / 8 and position L % 8 of it. Rows at or past `rows` read
// as zero (the buffer's range check; the row position is in the per-lane offset).
struct Stream {
    __amdgpu_buffer_rsrc_t rs;
    uint32_t voff[2];
    uint32_t tile_bytes;  // bytes between tiles (64 rows)

    __device__ __forceinline__ void init(const uint16_t *head, int64_t row_stride, int64_t rows, int wave, int lane) {
        rs = rsrc(head, rows * row_stride * 2);
        tile_bytes = (uint32_t)(TR * row_stride * 2);
#pragma unroll
        for (int i = 0; i < 2; ++i) {
            const int r = 8 * (2 * wave + i) + (lane >> 3);
            const int c = (lane & 7) ^ swz(r);
            voff[i] = (uint32_t)((r * row_stride + c * 8) * 2);
        }
    }
    __device__ __forceinline__ void issue(char *tile, int t, int wave) const {
        const uint32_t base = (uint32_t)t * tile_bytes;
#pragma unroll
        for (int i = 0; i < 2; ++i)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)(tile + (2 * wave + i) * 1024), 16,
                                                     voff[i] + base, 0, 0, 0);
    }
};

// 64 consecutive FP32 row values (LSE, rowsum(dO * O)) of a tile, loaded by lanes 0..15 of one wave.
struct RowStream {
    __amdgpu_buffer_rsrc_t rs;
    __device__ __forceinline__ void init(const float *row0, int64_t rows) { rs = rsrc(row0, rows * 4); }
    __device__ __forceinline__ void issue(char *dst, int t, int lane) const {
        if (lane < 16)
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void_t *)dst, 16, (uint32_t)(t * TR * 4 + lane * 16), 0,
                                                     0, 0);
    }
};

struct Head {
    int64_t heads, bs, hs, rs;
    __device__ __forceinline__ int64_t base(int64_t bh) const { return (bh / heads) * bs + (bh % heads) * hs; }
};

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// Four consecutive output values at element `idx` of an f32 or (bf16: RNE) BF16 array.
__device__ __forceinline__ void store4(void *base, int64_t idx, f32x4 v, int bf16) {
    if (bf16)
        *(u32x2 *)((uint16_t *)base + idx) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
    else
        *(f32x4 *)((float *)base + idx) = v;
}

// Workgroup (x, y) takes tile lin / heads-count of head lin % heads-count, lin = y * gridDim.x + x,
// so the first workgroups dispatched hold the costliest causal tile of every head.
__device__ __forceinline__ void grid_tile(int &tile, int64_t &bh) {
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    tile = (int)(lin / gridDim.y);
    bh = lin % gridDim.y;
}

__device__ __forceinline__ void wait_loads_and_reads() { __builtin_amdgcn_s_waitcnt(0x0070); }  // vmcnt(0) lgkmcnt(0)

// Streams n tiles: body(t, cur) with tile t in `cur`; loads of tile t+2 after the barrier that ends t.
template <typename Issue, typename Body>
__device__ __forceinline__ void stream_tiles(char *st0, char *st1, int n, Issue issue, Body body) {
    if (n <= 0) return;
    issue(st0, 0);
    wait_loads_and_reads();
    __syncthreads();
    if (n > 1) issue(st1, 1);
    int t = 0;
    for (; t + 1 < n; t += 2) {
        body(t, st0);
        wait_loads_and_reads();
        __syncthreads();
        if (t + 2 < n) issue(st0, t + 2);
        body(t + 1, st1);
        wait_loads_and_reads();
        __syncthreads();
        if (t + 3 < n) issue(st1, t + 3);
    }
    if (t < n) {
        body(t, st0);
        wait_loads_and_reads();
        __syncthreads();
    }
}

// NaN-propagating max (v_maximum3_f32 on gfx950: no operand canonicalisation, unlike fmaxf).
__device__ __forceinline__ float vmax(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Max over the lane pair l, l ^ 32 (the two halves of one query's keys): one v_permlane32_swap.
__device__ __forceinline__ float pair_max(float x) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
    return vmax(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// ------------------------------------------------------------------ forward

// Four waves per SIMD (at most 128 registers): the forward's max -> exp -> P.V chain is serial within
// a wave, so each 64-key tile is taken as two 32-key halves (one 16-register score block live, not
// two) and the row sum is added on the VALU instead of through an extra MFMA per chunk; four blocks
// of 32 KB LDS fit a CU. Measured against three waves with whole-tile softmax and the MFMA row sum:
// config 3 causal forward 36.4 -> 33.7 us.
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(4))) void flash2_fwd(const FlashArgs p) {
    __shared__ __attribute__((aligned(1024))) char st0[2 * TB];  // K tile, V tile
    __shared__ __attribute__((aligned(1024))) char st1[2 * TB];
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    int qb;
    int64_t bh;
    grid_tile(qb, bh);
    if (p.causal) qb = (int)gridDim.x - 1 - qb;  // the last query block sees every key block
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        ho{p.heads, p.o_bs, p.o_hs, p.o_rs};
    const uint16_t *Q = (const uint16_t *)p.Q + hq.base(bh);
    const uint16_t *K = (const uint16_t *)p.K + hk.base(bh);
    const uint16_t *V = (const uint16_t *)p.V + hk.base(bh);
    const int q = qb * RB + wave * 32 + (lane & 31);  // this lane's query
    const bool qok = q < p.sq;
    const int skv = (int)p.skv;
    const float c2 = p.scale * LOG2E;

    // Q^T as the B operand of S^T = K.Q^T: query q, d = 16 ks + 8h .. +7.
    u32x4 qf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const u32x4 v = ld16(Q + (qok ? (int64_t)q * p.q_rs + 16 * ks + 8 * h : 0));
        qf[ks] = qok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    // o[0], o[1]: O^T rows d 0..31, 32..63.
    f32x16 o[2] = {zero16(), zero16()};
    float m = -INFINITY;  // running max (log2 units) used by the probabilities
    float lsum = 0.f;     // this lane's share (its 32 of each tile's 64 keys) of the row sum

    const int kblocks = (int)((p.skv + TR - 1) / TR);
    const int nkb = p.causal ? min(kblocks, (qb * RB + RB - 1) / TR + 1) : kblocks;
    Stream sk, sv;
    sk.init(K, p.kv_rs, p.skv, wave, lane);
    sv.init(V, p.kv_rs, p.skv, wave, lane);
    const FragOff fo = frag_offsets(lane);
    stream_tiles(st0, st1, nkb, [&](char *st, int t) {
        sk.issue(st, t, wave);
        sv.issue(st + TB, t, wave);
    }, [&](int t, const char *st) {
        const char *kt = st, *vt = st + TB;
        const int k0 = t * TR;
        const bool edge = (p.causal && k0 + TR - 1 > qb * RB) || k0 + TR > skv;
        const int lim = p.causal ? min(skv - 1, q) : skv - 1;
        // Two halves of 32 keys: S^T block (keys 32kh + 8 (j / 4) + 4h + j % 4 of query q),
        // softmax, then its share of O^T += V^T . P^T.
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            f32x16 sh = zero16();
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) sh = mfma32(frag_rm_o(kt, fo, 32 * kh, ks), qf[ks], sh);
            if (edge) {
#pragma unroll
                for (int j = 0; j < 16; ++j) {
                    const int key = k0 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3);
                    sh[j] = key > lim ? -INFINITY : sh[j];
                }
            }
            float m4[4] = {sh[0], sh[1], sh[2], sh[3]};
#pragma unroll
            for (int j = 4; j < 16; ++j) m4[j & 3] = vmax(m4[j & 3], sh[j]);
            const float mx = pair_max(vmax(vmax(m4[0], m4[1]), vmax(m4[2], m4[3]))) * c2;
            if (__builtin_amdgcn_ballot_w64(mx > m + RESCALE) != 0) {
                const float mn = fmaxf(m, mx);
                const float alpha = mn == -INFINITY ? 1.f : __builtin_amdgcn_exp2f(m - mn);
                o[0] *= alpha;
                o[1] *= alpha;
                lsum *= alpha;
                m = mn;
            }
            const float nm = m == -INFINITY ? 0.f : -m;
#pragma unroll
            for (int j = 0; j < 16; ++j) sh[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sh[j], c2, nm));
            float ls4[4] = {sh[0], sh[1], sh[2], sh[3]};
#pragma unroll
            for (int j = 4; j < 16; ++j) ls4[j & 3] += sh[j];
            lsum += (ls4[0] + ls4[1]) + (ls4[2] + ls4[3]);
            u32x4 pf[2];
#pragma unroll
            for (int c = 0; c < 2; ++c)
                pf[c] = pack8(sh, 8 * c);
#pragma unroll
            for (int dh = 0; dh < 2; ++dh)
#pragma unroll
                for (int c = 0; c < 2; ++c) o[dh] = mfma32(frag_tr_o(vt, fo, 32 * dh, 16 * (2 * kh + c)), pf[c], o[dh]);
        }
    });
    const float l = lsum + __shfl_xor(lsum, 32, 64);
    if (qok) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
        const int64_t orow = ho.base(bh) + (int64_t)q * p.o_rs;
        // o[dh][j]: d = 32dh + 8 (j / 4) + 4h + j % 4
#pragma unroll
        for (int dh = 0; dh < 2; ++dh)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                store4(p.O, orow + 32 * dh + 8 * jj + 4 * h,
                       f32x4{o[dh][4 * jj], o[dh][4 * jj + 1], o[dh][4 * jj + 2], o[dh][4 * jj + 3]} * inv, p.o_bf16);
        if (h == 0 && p.lse) p.lse[bh * p.sq + q] = (m + __log2f(l)) * LN2;  // natural-log LSE
    }
}

// ------------------------------------------------------------------ backward: dQ (and rowsum(dO * O))

// One dQ block: query rows qb * RB .. + RB - 1 of head bh, LDS stages st0 and st1 of 2 TB bytes;
// -rowsum(dO * O) of its queries comes from the workspace (written by flash2_bwd_rows).
__device__ __forceinline__ void dq2_block(const FlashArgs &p, int qb, int64_t bh, char *st0, char *st1) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        hd{p.heads, p.do_bs, p.do_hs, p.do_rs}, ho{p.heads, p.o_bs, p.o_hs, p.o_rs};
    const uint16_t *Q = (const uint16_t *)p.Q + hq.base(bh);
    const uint16_t *K = (const uint16_t *)p.K + hk.base(bh);
    const uint16_t *V = (const uint16_t *)p.V + hk.base(bh);
    const uint16_t *dO = (const uint16_t *)p.dO + hd.base(bh);
    const int q = qb * RB + wave * 32 + (lane & 31);
    const bool qok = q < p.sq;
    const int skv = (int)p.skv;
    const float c2 = p.scale * LOG2E;

    // Q^T and dO^T as B operands: query q, d = 16 ks + 8h .. +7.
    u32x4 qf[4], of[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const u32x4 a = ld16(Q + (qok ? (int64_t)q * p.q_rs + 16 * ks + 8 * h : 0));
        const u32x4 b = ld16(dO + (qok ? (int64_t)q * p.do_rs + 16 * ks + 8 * h : 0));
        qf[ks] = qok ? a : u32x4{0u, 0u, 0u, 0u};
        of[ks] = qok ? b : u32x4{0u, 0u, 0u, 0u};
    }
    // rowsum(dO * O) of this query, stored negated by flash2_bwd_rows.
    const float dl = qok ? -p.dlt[bh * p.sq + q] : 0.f;
    const float nl2 = qok ? -p.lse[bh * p.sq + q] * LOG2E : 0.f;
    // dP^T accumulates from -rowsum (the same for all 16 rows of a lane's column), so the MFMA
    // leaves dP - rowsum(dO * O) and dS = P (dP - rowsum) is one multiply.
    const float ndl = -dl;
    const f32x16 ndl16 = {ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl, ndl};
    f32x16 dq[2] = {zero16(), zero16()};

    const int kblocks = (int)((p.skv + TR - 1) / TR);
    const int nkb = p.causal ? min(kblocks, (qb * RB + RB - 1) / TR + 1) : kblocks;
    Stream sk, sv;
    sk.init(K, p.kv_rs, p.skv, wave, lane);
    sv.init(V, p.kv_rs, p.skv, wave, lane);
    const FragOff fo = frag_offsets(lane);
    stream_tiles(st0, st1, nkb, [&](char *st, int t) {
        sk.issue(st, t, wave);
        sv.issue(st + TB, t, wave);
    }, [&](int t, const char *st) {
        const char *kt = st, *vt = st + TB;
        // One 32-key half of the tile at a time: S^T = K.Q^T and dP^T = V.dO^T (block of keys
        // 32kh + 8 (j / 4) + 4h + j % 4), P^T = exp2(S^T scale log2 e - LSE log2 e), zero past the
        // query (causal) and past seq_kv (K and V rows there are zero, but an unmasked probability
        // could overflow into 0 * inf): masked scores become -inf before the exponential, in a
        // wave-uniform branch taken only by the tiles that hold such keys. dS^T = P^T (dP^T - rowsum)
        // then feeds dQ^T (d x queries) += K^T (d x keys) . dS^T (keys x queries).
        const int k0 = t * TR;
        const bool edge = (p.causal && k0 + TR - 1 > qb * RB) || k0 + TR > skv;
        const int lim = p.causal ? min(skv - 1, q) : skv - 1;
#pragma unroll
        for (int kh = 0; kh < 2; ++kh) {
            f32x16 sh = zero16(), dph = ndl16;
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                sh = mfma32(frag_rm_o(kt, fo, 32 * kh, ks), qf[ks], sh);
                dph = mfma32(frag_rm_o(vt, fo, 32 * kh, ks), of[ks], dph);
            }
            if (edge) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    sh[j] = k0 + 32 * kh + 8 * (j >> 2) + 4 * h + (j & 3) > lim ? -INFINITY : sh[j];
            }
#pragma unroll
            for (int j = 0; j < 16; ++j) dph[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(sh[j], c2, nl2)) * dph[j];
#pragma unroll
            for (int c = 0; c < 2; ++c) {
                const u32x4 df = pack8(dph, 8 * c);
#pragma unroll
                for (int dh = 0; dh < 2; ++dh) dq[dh] = mfma32(frag_tr_o(kt, fo, 32 * dh, 16 * (2 * kh + c)), df, dq[dh]);
            }
        }
    });
    if (qok) {
        const int64_t row = hq.base(bh) + (int64_t)q * p.q_rs;
#pragma unroll
        for (int dh = 0; dh < 2; ++dh)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                store4(p.dQ, row + 32 * dh + 8 * jj + 4 * h,
                       f32x4{dq[dh][4 * jj], dq[dh][4 * jj + 1], dq[dh][4 * jj + 2], dq[dh][4 * jj + 3]} * p.scale,
                       p.grad_bf16);
    }
}


// ------------------------------------------------------------------ backward: dK, dV

constexpr int DKDV2_STAGE = 2 * TB + 2 * TR * 4;  // Q tile, dO tile, -LSE log2 e and -rowsum(dO * O) rows

// One dK/dV block: keys kb * RB .. + RB - 1 of head bh, LDS stages st0 and st1 of DKDV2_STAGE bytes.
__device__ __forceinline__ void dkdv2_block(const FlashArgs &p, int kb, int64_t bh, char *st0, char *st1) {
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int h = lane >> 5;
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        hd{p.heads, p.do_bs, p.do_hs, p.do_rs};
    const uint16_t *Q = (const uint16_t *)p.Q + hq.base(bh);
    const uint16_t *K = (const uint16_t *)p.K + hk.base(bh);
    const uint16_t *V = (const uint16_t *)p.V + hk.base(bh);
    const uint16_t *dO = (const uint16_t *)p.dO + hd.base(bh);
    const int key = kb * RB + wave * 32 + (lane & 31);  // this lane's key
    const bool kok = key < p.skv;
    const float c2 = p.scale * LOG2E;

    // K^T and V^T as B operands of S = Q.K^T and dP = dO.V^T: key, d = 16 ks + 8h .. +7.
    u32x4 kf[4], vf[4];
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
        const int64_t off = kok ? (int64_t)key * p.kv_rs + 16 * ks + 8 * h : 0;
        const u32x4 a = ld16(K + off), b = ld16(V + off);
        kf[ks] = kok ? a : u32x4{0u, 0u, 0u, 0u};
        vf[ks] = kok ? b : u32x4{0u, 0u, 0u, 0u};
    }
    f32x16 dk[2] = {zero16(), zero16()}, dv[2] = {zero16(), zero16()};

    const int qblocks = (int)((p.sq + TR - 1) / TR);
    const int qb0 = p.causal ? min(qblocks, kb * RB / TR) : 0;
    Stream sq_, sd;
    sq_.init(Q, p.q_rs, p.sq, wave, lane);
    sd.init(dO, p.do_rs, p.sq, wave, lane);
    RowStream rl, rd;  // rows flash2_bwd_rows left in the workspace
    rl.init(p.dlt + p.bh * p.sq + bh * p.sq, p.sq);
    rd.init(p.dlt + bh * p.sq, p.sq);
    const FragOff fo = frag_offsets(lane);
    stream_tiles(st0, st1, qblocks - qb0, [&](char *st, int t) {
        sq_.issue(st, qb0 + t, wave);
        sd.issue(st + TB, qb0 + t, wave);
        if (wave == 0) rl.issue(st + 2 * TB, qb0 + t, lane);
        if (wave == 1) rd.issue(st + 2 * TB + TR * 4, qb0 + t, lane);
    }, [&](int t, const char *st) {
        const char *qt = st, *dot = st + TB;
        const float *nl2 = (const float *)(st + 2 * TB), *ndl = nl2 + TR;
        const int q0 = (qb0 + t) * TR;
        const bool diag = p.causal && q0 < kb * RB + RB;
        const int kq = key - q0;  // this key against query row r of the tile: masked when kq > r
        // One 32-query half of the tile at a time (S, dP, P, dS of half qh live together, not both
        // halves), which keeps the kernel within three waves' registers per SIMD.
#pragma unroll
        for (int qh = 0; qh < 2; ++qh) {
            // S = Q.K^T and dP = dO.V^T: queries 32qh + 8 (j / 4) + 4h + j % 4 of this lane's key;
            // dP accumulates from -rowsum(dO * O) of those queries.
            f32x16 sv = zero16(), dpv;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const f32x4 v = *(const f32x4 *)(ndl + 32 * qh + 8 * jj + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) dpv[4 * jj + e] = v[e];
            }
#pragma unroll
            for (int ks = 0; ks < 4; ++ks) {
                sv = mfma32(frag_rm_o(qt, fo, 32 * qh, ks), kf[ks], sv);
                dpv = mfma32(frag_rm_o(dot, fo, 32 * qh, ks), vf[ks], dpv);
            }
            // P = exp2(S scale log2 e - LSE log2 e), zero for queries before this key (causal: the
            // score becomes -inf in a wave-uniform branch that only diagonal tiles take); rows past
            // seq_q have zero Q and dO (and read as zero from the workspace rows): they add nothing
            // to dK or dV. dS = P (dP - rowsum).
            if (diag) {
#pragma unroll
                for (int j = 0; j < 16; ++j)
                    sv[j] = kq > 32 * qh + 8 * (j >> 2) + 4 * h + (j & 3) ? -INFINITY : sv[j];
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const f32x4 lv = *(const f32x4 *)(nl2 + 32 * qh + 8 * jj + 4 * h);
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                    const int j = 4 * jj + e;
                    const float pr = __builtin_amdgcn_exp2f(__builtin_fmaf(sv[j], c2, lv[e]));
                    sv[j] = pr;
                    dpv[j] = pr * dpv[j];
                }
            }
            // dV^T (d x keys) += dO^T (d x queries) . P;  dK^T += Q^T . dS  (query chunks 2qh, 2qh + 1)
#pragma unroll
            for (int cc = 0; cc < 2; ++cc) {
                const u32x4 pf = pack8(sv, 8 * cc), df = pack8(dpv, 8 * cc);
#pragma unroll
                for (int dh = 0; dh < 2; ++dh) {
                    dv[dh] = mfma32(frag_tr_o(dot, fo, 32 * dh, 16 * (2 * qh + cc)), pf, dv[dh]);
                    dk[dh] = mfma32(frag_tr_o(qt, fo, 32 * dh, 16 * (2 * qh + cc)), df, dk[dh]);
                }
            }
        }
    });
    if (kok) {
        const int64_t row = hk.base(bh) + (int64_t)key * p.kv_rs;
#pragma unroll
        for (int dh = 0; dh < 2; ++dh)
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
                const int d = 32 * dh + 8 * jj + 4 * h;
                store4(p.dK, row + d,
                       f32x4{dk[dh][4 * jj], dk[dh][4 * jj + 1], dk[dh][4 * jj + 2], dk[dh][4 * jj + 3]} * p.scale,
                       p.grad_bf16);
                store4(p.dV, row + d, f32x4{dv[dh][4 * jj], dv[dh][4 * jj + 1], dv[dh][4 * jj + 2], dv[dh][4 * jj + 3]},
                       p.grad_bf16);
            }
    }
}


// The workspace rows of every query: -rowsum(dO * O) at dlt[row] and -LSE log2 e at
// dlt[bh seq + row], 8 lanes per row (8 columns each: 32 bytes of O, 16 of dO), for
// flash2_bwd_fused.
__global__ __launch_bounds__(256) void flash2_bwd_rows(const FlashArgs p) {
    const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int c = threadIdx.x & 7;
    if (row >= p.bh * p.sq) return;  // whole 8-lane groups leave together
    const int64_t bh = row / p.sq, q = row % p.sq;
    const Head hd{p.heads, p.do_bs, p.do_hs, p.do_rs}, ho{p.heads, p.o_bs, p.o_hs, p.o_rs};
    auto lo = [](uint32_t w) { return __uint_as_float(w << 16); };
    auto hi = [](uint32_t w) { return __uint_as_float(w & 0xffff0000u); };
    const int64_t oi = ho.base(bh) + q * p.o_rs + 8 * c;
    f32x4 o0, o1;
    if (p.o_bf16) {
        const u32x4 ob = *(const u32x4 *)((const uint16_t *)p.O + oi);
        o0 = f32x4{lo(ob[0]), hi(ob[0]), lo(ob[1]), hi(ob[1])};
        o1 = f32x4{lo(ob[2]), hi(ob[2]), lo(ob[3]), hi(ob[3])};
    } else {
        o0 = *(const f32x4 *)((const float *)p.O + oi);
        o1 = *(const f32x4 *)((const float *)p.O + oi + 4);
    }
    const u32x4 g = *(const u32x4 *)((const uint16_t *)p.dO + hd.base(bh) + q * p.do_rs + 8 * c);
    float s = lo(g[0]) * o0[0] + hi(g[0]) * o0[1] + lo(g[1]) * o0[2] + hi(g[1]) * o0[3] + lo(g[2]) * o1[0] +
              hi(g[2]) * o1[1] + lo(g[3]) * o1[2] + hi(g[3]) * o1[3];
#pragma unroll
    for (int w = 1; w < 8; w <<= 1) s += __shfl_xor(s, w, 64);
    if (c == 0) {
        p.dlt[row] = -s;
        p.dlt[p.bh * p.sq + row] = -p.lse[row] * LOG2E;
    }
}

// The backward for grids with as many key blocks as query blocks: block j computes dQ of query
// block j, then dK and dV of key block j. Under the causal mask the two parts' tile counts add up
// to the same number for every block. Three waves per SIMD (168 registers; 32-key or 32-query halves
// and per-lane fragment offsets keep both parts within them): config 3 causal backward 105 -> 101 us,
// non-causal 173 -> 158 us against two waves.
__global__ __launch_bounds__(NTH) __attribute__((amdgpu_waves_per_eu(3))) void flash2_bwd_fused(const FlashArgs p) {
    __shared__ __attribute__((aligned(1024))) char st0[DKDV2_STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[DKDV2_STAGE];
    int j;
    int64_t bh;
    grid_tile(j, bh);
    dq2_block(p, j, bh, st0, st1);
    __syncthreads();  // the dQ part's last LDS reads before the dK/dV part's first writes
    dkdv2_block(p, j, bh, st0, st1);
}

}  // namespace

// The BF16 kernels above need 16-byte aligned operand rows (checked by flash_supported) and 32-bit
// buffer offsets: every operand's rows of one head within 2 GiB.
bool flash2_applicable(const FlashArgs &p, bool backward) {
    auto fits = [](int64_t rows, int64_t rs) { return rows * rs * 2 < (1ll << 31); };
    bool ok = fits(p.skv, p.kv_rs);
    if (backward) ok = ok && fits(p.sq, p.q_rs) && fits(p.sq, p.do_rs) && p.sq * 4 < (1ll << 31);
    return ok;
}

it_status launch_flash2_fwd(hipStream_t s, const FlashArgs &p) {
    const int64_t qblocks = (p.sq + RB - 1) / RB;
    if (qblocks > 0x7fffffff || p.bh > 65535) return fail(IT_ERR_DIMS, "flash attention: grid too large");
    hipLaunchKernelGGL(flash2_fwd, dim3((unsigned)qblocks, (unsigned)p.bh), dim3(NTH), 0, s, p);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_flash2_bwd(hipStream_t s, const FlashArgs &p) {
    const int64_t blocks = (p.sq + RB - 1) / RB;  // query blocks = key blocks (equal lengths)
    if (blocks > 0x7fffffff || p.bh > 65535) return fail(IT_ERR_DIMS, "flash attention backward: grid too large");
    // The workspace rows of every query first, then one kernel of balanced dQ + dK/dV blocks.
    const int64_t rows = p.bh * p.sq;
    hipLaunchKernelGGL(flash2_bwd_rows, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, p);
    hipLaunchKernelGGL(flash2_bwd_fused, dim3((unsigned)blocks, (unsigned)p.bh), dim3(NTH), 0, s, p);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
