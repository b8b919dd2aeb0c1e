// Fused attention contractions for head_dim 64 on gfx950 MFMA ("flash" form: S and P never reach
// HBM). Same mathematics as ops::attention / attention_backward_recompute
// (src/ops/attention.rs:286-377, src/train/helpers.rs:120-193): S = scale * Q.K^T, causal -inf above
// the diagonal, P = softmax(S) per row, O = P.V; backward dV = P^T.dO, dP = dO.V^T,
// dS = P * (dP - rowsum(dP * P)), dQ = scale * dS.K, dK = scale * dS^T.Q. The softmax runs online
// over 64-key blocks (running max and sum, rescaling the partial output), and the backward uses
// rowsum(dP * P) = rowsum(dO * O) and P = exp(S - LSE) with the row log-sum-exp saved by the forward.
//
// Layout choice: every block owns 64 rows (queries or keys), one wave per 16 rows. Products are
// arranged so that a lane's accumulator values belong to one query (S^T = K.Q^T puts the query on
// the lane's column), which keeps the softmax statistics to two cross-lane shuffles and lets the
// probabilities feed the next MFMA straight from the accumulators:
//   forward : S^T = K.Q^T,       O^T += V^T.P^T
//   dK / dV : S = Q.K^T, dP = dO.V^T (keys on the lane's column), dV += P^T.dO, dK += dS^T.Q
//   dQ      : S^T = K.Q^T, dP^T = V.dO^T,                          dQ^T += K^T.dS^T
// The backward is deterministic: dK/dV and dQ come from two kernels instead of atomics.
// BF16 operands accumulate in FP32; P and dS are rounded to BF16 before their MFMA. When a
// fragment comes from accumulators (P, dS), a BF16 lane group g holds keys {4g..4g+3} and
// {16+4g..16+4g+3} of a 32-key chunk, and the LDS operand it meets is read with the same split.
#include <algorithm>
#include <cmath>

#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int HD = 64;   // head dim
constexpr int TR = 64;   // rows per tile
constexpr int NTH = 256;

template <typename T>
struct FE;
template <>
struct FE<float> {
    static constexpr int KC = 16;  // k per fragment chunk
    static constexpr int VEC = 4;  // elements per 16 bytes
};
template <>
struct FE<uint16_t> {
    static constexpr int KC = 32;
    static constexpr int VEC = 8;
};

template <typename T>
constexpr int pitch() { return HD * (int)sizeof(T) + 16; }  // LDS bytes per tile row
template <typename T>
constexpr int tile_bytes() { return TR * pitch<T>(); }

struct Head {
    int64_t heads, bs, hs, rs;
    __device__ __forceinline__ int64_t base(int64_t bh) const { return (bh / heads) * bs + (bh % heads) * hs; }
};

__device__ __forceinline__ u32x4 ld16(const void *p) { return *(const u32x4 *)p; }

// 64x64 tiles move global -> registers -> LDS in units of 4 rows x 16 bytes (4 x VEC elements).
// From one unit a thread can write both LDS layouts: row-major ([row][d]) and transposed ([d][row],
// for operands whose MFMA k index is the tile row), so a tensor needed both ways is read from HBM
// once.
//
// Unit u covers rows 4rg..4rg+3 and 16-byte column cc. FP32: cc is fastest, so the 16 lanes that
// share rg load 256 contiguous bytes of each row (the memory pipeline's cost follows the lanes'
// addresses in lane order), and the 16-byte units of LDS row r are XOR-swizzled by (r >> 4) & 3
// (swz): the row-major writes of 16 lanes fill one row, the transposed writes land in rows 4cc + j
// at 16 distinct bank groups, and the fragment reads of 16 consecutive rows stay conflict-free.
// BF16: a tile that is stored transposed takes consecutive rg in consecutive lanes, so the
// transposed writes of neighbouring lanes fill one LDS row side by side; a tile stored only
// row-major keeps cc fastest.
template <typename T>
__device__ __forceinline__ int swz(int row, int u) {
    if constexpr (sizeof(T) == 4)
        return u ^ ((row >> 4) & 3);
    else
        return u;
}

template <typename T>
struct Unit4 {
    static constexpr int VEC = FE<T>::VEC;
    static constexpr int CPR = HD / VEC;   // 16-byte columns per row
    static constexpr int RGS = TR / 4;     // row groups
    u32x4 r[4];

    __device__ __forceinline__ static void decode(int u, bool rg_fast, int &rg, int &cc) {
        const bool rf = rg_fast && sizeof(T) == 2;
        rg = rf ? u % RGS : u / CPR;
        cc = rf ? u / RGS : u % CPR;
    }

    __device__ __forceinline__ void load(const T *m, int64_t rs, int row0, int rows, int u, bool rg_fast) {
        int rg, cc;
        decode(u, rg_fast, rg, cc);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const int row = row0 + rg * 4 + q;
            const bool ok = row < rows;
            const u32x4 v = ld16(m + (ok ? (int64_t)row * rs + cc * VEC : 0));
            r[q] = ok ? v : u32x4{0u, 0u, 0u, 0u};
        }
    }
    __device__ __forceinline__ void store_rows(char *lds, int u, bool rg_fast) const {
        constexpr int P = pitch<T>();
        int rg, cc;
        decode(u, rg_fast, rg, cc);
#pragma unroll
        for (int q = 0; q < 4; ++q) *(u32x4 *)(lds + (rg * 4 + q) * P + swz<T>(rg * 4 + q, cc) * 16) = r[q];
    }
    __device__ __forceinline__ void store_cols(char *lds, int u, bool rg_fast) const {
        constexpr int P = pitch<T>();
        int rg, cc;
        decode(u, rg_fast, rg, cc);
        const u32x4 &v0 = r[0], &v1 = r[1], &v2 = r[2], &v3 = r[3];
        if constexpr (sizeof(T) == 4) {
            // 4 rows x 4 columns -> LDS rows 4cc+j, columns 4rg..4rg+3
#pragma unroll
            for (int j = 0; j < 4; ++j)
                *(u32x4 *)(lds + (cc * 4 + j) * P + swz<T>(cc * 4 + j, rg) * 16) = u32x4{v0[j], v1[j], v2[j], v3[j]};
        } else {
            // 4 rows x 8 bf16 columns -> LDS rows 8cc+j, columns 4rg..4rg+3 (8 bytes)
#pragma unroll
            for (int d = 0; d < 4; ++d) {
                u32x2 lo, hi;
                lo[0] = (v0[d] & 0xffffu) | (v1[d] << 16);
                lo[1] = (v2[d] & 0xffffu) | (v3[d] << 16);
                hi[0] = (v0[d] >> 16) | (v1[d] & 0xffff0000u);
                hi[1] = (v2[d] >> 16) | (v3[d] & 0xffff0000u);
                *(u32x2 *)(lds + (cc * 8 + 2 * d) * P + rg * 8) = lo;
                *(u32x2 *)(lds + (cc * 8 + 2 * d + 1) * P + rg * 8) = hi;
            }
        }
    }
};

// Two 64x64 row tiles (tensors 0 and 1, same row blocks) streamed through LDS with two register
// sets, so the loads of block t+2 are in flight while block t is computed and block t+1 waits in
// registers. FP32: 256 units per tile, every thread moves one unit of each; BF16: 128 units, waves
// 0-1 move tensor 0 and waves 2-3 tensor 1. Each tensor goes to LDS row-major, transposed or both
// (an offset < 0 skips a layout). Optionally two per-row FP32 vectors (aux) ride along, scaled, for
// rows blk*64 + tid (tid < 64), into `aux_off`.
template <typename T, int NT = NTH>
struct TilePair {
    static constexpr int PER_TILE = TR * HD / (4 * FE<T>::VEC);
    static constexpr int SLOTS = 2 * PER_TILE >= NT ? 2 * PER_TILE / NT : 1;
    static constexpr bool ALL = 2 * PER_TILE >= NT;  // every thread moves units
    const T *m[2];
    int64_t rs[2];
    int rows[2];
    int off_rows[2], off_cols[2];
    const float *aux[2] = {nullptr, nullptr};
    float aux_scale[2] = {1.f, 1.f};
    int aux_off = -1, aux_rows = 0;
    int tid;
    Unit4<T> set0[SLOTS], set1[SLOTS];
    float x0[2], x1[2];

    __device__ __forceinline__ int tensor(int s) const { return SLOTS == 2 ? s : (tid >= PER_TILE ? 1 : 0); }
    __device__ __forceinline__ int unit() const { return SLOTS == 2 ? tid : tid % PER_TILE; }

    template <int SET>
    __device__ __forceinline__ void load(int blk) {
        Unit4<T> *r = SET ? set1 : set0;
        float *x = SET ? x1 : x0;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            if (!ALL && tid >= 2 * PER_TILE) break;
            const int t = tensor(s);
            r[s].load(m[t], rs[t], blk * TR, rows[t], unit(), off_cols[t] >= 0);
        }
        if (aux_off >= 0 && tid < TR) {
            const int row = blk * TR + tid;
#pragma unroll
            for (int a = 0; a < 2; ++a) x[a] = row < aux_rows ? aux[a][row] * aux_scale[a] : 0.f;
        }
    }
    template <int SET>
    __device__ __forceinline__ void store(char *stage) const {
        const Unit4<T> *r = SET ? set1 : set0;
        const float *x = SET ? x1 : x0;
#pragma unroll
        for (int s = 0; s < SLOTS; ++s) {
            if (!ALL && tid >= 2 * PER_TILE) break;
            const int t = tensor(s);
            const bool rg_fast = off_cols[t] >= 0;
            if (off_rows[t] >= 0) r[s].store_rows(stage + off_rows[t], unit(), rg_fast);
            if (rg_fast) r[s].store_cols(stage + off_cols[t], unit(), rg_fast);
        }
        if (aux_off >= 0 && tid < TR) {
            ((float *)(stage + aux_off))[tid] = x[0];
            ((float *)(stage + aux_off + TR * 4))[tid] = x[1];
        }
    }
};

// Runs body(t, stage) for t = 0..n-1 on row blocks b0 + t, block t's tiles in LDS stage t % 2.
// Block t+2 is loaded as body t starts and written to LDS after body t+1, so its loads have two
// blocks of compute to land.
template <typename TP, typename Body>
__device__ __forceinline__ void pipelined(TP &tp, char *smem, int stage_bytes, int b0, int n, Body body) {
    if (n > 0) {
        tp.template load<0>(b0);
        tp.template store<0>(smem);
    }
    if (n > 1) tp.template load<1>(b0 + 1);
    __syncthreads();
    for (int t = 0; t < n; t += 2) {
        if (t + 2 < n) tp.template load<0>(b0 + t + 2);
        body(t, (const char *)smem);
        if (t + 1 < n) tp.template store<1>(smem + stage_bytes);
        __syncthreads();
        if (t + 1 >= n) break;
        if (t + 3 < n) tp.template load<1>(b0 + t + 3);
        body(t + 1, (const char *)(smem + stage_bytes));
        if (t + 2 < n) tp.template store<0>(smem);
        __syncthreads();
    }
}

// Fragment of LDS tile row `row`, contiguous k chunk c (lane group g).
template <typename T>
__device__ __forceinline__ u32x4 frag_c(const char *tile, int row, int c, int g) {
    // (c * KC + g * VEC) elements = 16-byte unit 4c + g, for both element types
    return *(const u32x4 *)(tile + row * pitch<T>() + swz<T>(row, 4 * c + g) * 16);
}

// Fragment whose k assignment matches an accumulator-derived operand: FP32 chunk c = keys
// 16c + 4g..+3 (same as frag_c); BF16 chunk c = keys 32c + 4g..+3 and 32c + 16 + 4g..+3.
template <typename T>
__device__ __forceinline__ u32x4 frag_s(const char *tile, int row, int c, int g) {
    if constexpr (sizeof(T) == 4) {
        return frag_c<T>(tile, row, c, g);
    } else {
        const char *p = tile + row * pitch<T>();
        const u32x2 lo = *(const u32x2 *)(p + (32 * c + 4 * g) * 2);
        const u32x2 hi = *(const u32x2 *)(p + (32 * c + 16 + 4 * g) * 2);
        return u32x4{lo[0], lo[1], hi[0], hi[1]};
    }
}

// Operand fragment from accumulator blocks (rows 4g + r of 16-row blocks): FP32 uses block c,
// BF16 packs blocks 2c and 2c+1.
template <typename T>
__device__ __forceinline__ u32x4 frag_acc(const f32x4 *blk, int c) {
    if constexpr (sizeof(T) == 4) {
        return __builtin_bit_cast(u32x4, blk[c]);
    } else {
        const f32x4 a = blk[2 * c], b = blk[2 * c + 1];
        return u32x4{pack_bf16x2(a[0], a[1]), pack_bf16x2(a[2], a[3]), pack_bf16x2(b[0], b[1]),
                     pack_bf16x2(b[2], b[3])};
    }
}

__device__ __forceinline__ float xmax(float v) {
    v = fmaxf(v, __shfl_xor(v, 16, 64));
    return fmaxf(v, __shfl_xor(v, 32, 64));
}
__device__ __forceinline__ float xsum(float v) {
    v += __shfl_xor(v, 16, 64);
    return v + __shfl_xor(v, 32, 64);
}

// 2^x on the hardware unit (v_exp_f32, 1 ulp). Scores are carried in the log2 domain: they are
// multiplied by scale * log2(e) once, so every probability is one subtraction and one exp2.
__device__ __forceinline__ float exp2_fast(float x) { return __builtin_amdgcn_exp2f(x); }
constexpr float LOG2E = 1.4426950408889634f;
constexpr float LN2 = 0.6931471805599453f;

// Work order across the whole grid. Workgroups are dispatched in linear order (x fastest), and a
// causal row or column block's cost grows with its index, so block (x, y) takes tile
// lin / heads-count of head lin % heads-count, lin = y * gridDim.x + x: the first wave of
// workgroups holds the costliest tile of every head, the last the cheapest (longest-first
// scheduling), and a head's tiles stay on one XCD when the head count is a multiple of 8.
__device__ __forceinline__ void grid_tile(int &tile, int64_t &bh) {
    const int64_t lin = (int64_t)blockIdx.y * gridDim.x + blockIdx.x;
    tile = (int)(lin / gridDim.y);
    bh = lin % gridDim.y;
}

// ------------------------------------------------------------------ forward

// WG wave groups: with WG = 2 a block runs 8 waves, and wave w's 16 rows are shared by waves w and
// w + 4, each taking two of every tile's four 16-column blocks (grp = wave / 4 picks which). The
// two groups read the same LDS tiles; their partial results meet through LDS at the end, group 1's
// added to group 0's in a fixed order. A launch whose blocks fit one round on the CUs thereby runs
// twice the waves, each with half the work per tile.
constexpr int group_of(int wave8) { return wave8 >> 2; }

// Group 1 hands `n` floats per lane to group 0 through LDS ([job][n][lane], conflict-free), each
// wave at the slot of its 16-row job; call after the tile loop's final barrier, by every thread.
// Returns false for group 1 (done).
template <int N>
__device__ __forceinline__ bool hand_over(char *smem, int grp, int job, int lane, float (&v)[N]) {
    float *x = (float *)smem + job * N * 64 + lane;
    if (grp == 1) {
#pragma unroll
        for (int i = 0; i < N; ++i) x[i * 64] = v[i];
    }
    __syncthreads();
    if (grp == 1) return false;
#pragma unroll
    for (int i = 0; i < N; ++i) v[i] = x[i * 64];
    return true;
}

template <typename T, int WG>
__global__ __launch_bounds__(NTH * WG) void flash_fwd(const FlashArgs p) {
    constexpr int KT = tile_bytes<T>();      // K tile [keys][d]
    constexpr int STAGE = 2 * KT;            // + V^T tile [d][keys]
    constexpr int NC = HD / FE<T>::KC;       // d chunks
    constexpr int MBG = 4 / WG;              // 16-key blocks per group and tile
    constexpr int PCG = TR / FE<T>::KC / WG; // P chunks per group and tile
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, grp = group_of(tid >> 6);
    const int ql = lane & 15, g = lane >> 4;
    int x;
    int64_t bh;
    grid_tile(x, bh);
    const int nq = (int)gridDim.x, kblocks = (p.skv + TR - 1) / TR;
    // The block's 64 rows are four 16-row jobs: jobs 0-1 rows ra.., jobs 2-3 rows rz.. . Plain:
    // one query block (causal: last-first, as the last query block sees every key block). Causal
    // with two groups: rows 32h.. of query blocks i and nq - 1 - i (block x = 2i + h; the middle
    // block of an odd count takes both halves of its own), and group 1's wave w takes job
    // (w + 2) & 3, so each SIMD holds one wave of each query block: (i + 1 + nq - i) / 2 key tiles
    // of work on every SIMD instead of up to nq.
    const bool paired = WG == 2 && p.causal;
    const int job = paired && grp == 1 ? (wave + 2) & 3 : wave;
    int qa, qz, ra, rz;
    if (paired && x < nq / 2 * 2) {
        qa = x >> 1;
        qz = nq - 1 - qa;
        ra = qa * TR + (x & 1) * 32;
        rz = qz * TR + (x & 1) * 32;
    } else {
        qa = qz = paired ? nq / 2 : (p.causal ? nq - 1 - x : x);
        ra = qa * TR;
        rz = ra + 32;
    }
    const int qb = job < 2 ? qa : qz;
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        ho{p.heads, p.o_bs, p.o_hs, p.o_rs};
    const T *Q = (const T *)p.Q + hq.base(bh);
    const T *K = (const T *)p.K + hk.base(bh);
    const T *V = (const T *)p.V + hk.base(bh);
    float *O = (float *)p.O + ho.base(bh);
    const float c2 = p.scale * LOG2E;
    const int q = (job < 2 ? ra : rz) + (job & 1) * 16 + ql;  // this lane's query
    const bool qok = q < p.sq;

    u32x4 qf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const u32x4 v = ld16(Q + (qok ? (int64_t)q * p.q_rs + c * FE<T>::KC + g * FE<T>::VEC : 0));
        qf[c] = qok ? v : u32x4{0u, 0u, 0u, 0u};
    }
    f32x4 o[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] = f32x4{0.f, 0.f, 0.f, 0.f};
    float m = -INFINITY, l = 0.f;

    const int nkb = p.causal ? min(kblocks, qb + 1) : kblocks;               // this wave's key blocks
    const int nkb_all = p.causal ? min(kblocks, max(qa, qz) + 1) : kblocks;  // the block's
    TilePair<T, NTH * WG> tp;
    tp.tid = tid;
    tp.m[0] = K;  // K row-major
    tp.m[1] = V;  // V transposed
    tp.rs[0] = tp.rs[1] = p.kv_rs;
    tp.rows[0] = tp.rows[1] = (int)p.skv;
    tp.off_rows[0] = 0;
    tp.off_cols[0] = -1;
    tp.off_rows[1] = -1;
    tp.off_cols[1] = KT;
    pipelined(tp, smem, STAGE, 0, nkb_all, [&](int kb, const char *kt) {
        if (kb >= nkb) return;  // past this wave's causal range (wave-uniform)
        const char *vt = kt + KT;
        // S^T blocks: keys 16mb + 4g + r of this tile (mb = grp * MBG + i), query q.
        f32x4 s[MBG];
#pragma unroll
        for (int i = 0; i < MBG; ++i) {
            const int mb = grp * MBG + i;
            s[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) mma16<T>(s[i], frag_c<T>(kt, mb * 16 + ql, c, g), qf[c]);
        }
        // Scores to the log2 domain; keys past the diagonal (causal) or past seq_kv are -inf. Only
        // the last key block of a row block can hold such keys.
        float mx = -INFINITY;
        if (kb == nkb - 1 && (p.causal || p.skv % TR != 0)) {
#pragma unroll
            for (int i = 0; i < MBG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kb * TR + (grp * MBG + i) * 16 + g * 4 + r;
                    const bool dead = key >= p.skv || (p.causal && key > q);
                    s[i][r] = dead ? -INFINITY : s[i][r] * c2;
                    mx = fmaxf(mx, s[i][r]);
                }
        } else {
#pragma unroll
            for (int i = 0; i < MBG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    s[i][r] *= c2;
                    mx = fmaxf(mx, s[i][r]);
                }
        }
        const float mnew = fmaxf(m, xmax(mx));
        const float msafe = mnew == -INFINITY ? 0.f : mnew;
        const float alpha = exp2_fast(m - msafe);
        float ls = 0.f;
#pragma unroll
        for (int i = 0; i < MBG; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float e = exp2_fast(s[i][r] - msafe);
                s[i][r] = e;
                ls += e;
            }
        l = l * alpha + xsum(ls);
        m = mnew;
#pragma unroll
        for (int d = 0; d < 4; ++d) o[d] *= alpha;
        // O^T (d x q) += V^T (d x keys) . P^T (keys x q), over this group's keys
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int c = 0; c < PCG; ++c)
                mma16<T>(o[d], frag_s<T>(vt, d * 16 + ql, grp * PCG + c, g), frag_acc<T>(s, c));
    });
    if constexpr (WG == 2) {
        // Each group ran the online softmax over its own keys: merge (m, l, O) at the larger max.
        float v[18];
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[d * 4 + r] = o[d][r];
        v[16] = m;
        v[17] = l;
        float mine[18];
#pragma unroll
        for (int i = 0; i < 18; ++i) mine[i] = v[i];
        if (!hand_over<18>(smem, grp, job, lane, v)) return;
        const float m1 = v[16], mn = fmaxf(m, m1), ms = mn == -INFINITY ? 0.f : mn;
        const float a0 = exp2_fast(m - ms), a1 = exp2_fast(m1 - ms);
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) o[d][r] = mine[d * 4 + r] * a0 + v[d * 4 + r] * a1;
        l = l * a0 + v[17] * a1;
        m = mn;
    }
    if (qok) {
        const float inv = l > 0.f ? 1.f / l : 0.f;
#pragma unroll
        for (int d = 0; d < 4; ++d) *(f32x4 *)(O + (int64_t)q * p.o_rs + d * 16 + g * 4) = o[d] * inv;
        if (g == 0 && p.lse) p.lse[bh * p.sq + q] = (m + __log2f(l)) * LN2;  // natural-log LSE
    }
}


// ------------------------------------------------------------------ backward


// dK, dV for 64 keys per block (16 per wave), looping over the query blocks that see them. WG = 2:
// each wave group takes half of every query tile's rows (see flash_fwd).
template <typename T>
constexpr int dkdv_lds() { return 2 * (4 * tile_bytes<T>() + 2 * TR * 4); }

template <typename T, int WG>
__device__ __forceinline__ void dkdv_block(const FlashArgs &p, int kb, int64_t bh, char *smem) {
    constexpr int T_ = tile_bytes<T>();
    constexpr int STAGE = 4 * T_ + 2 * TR * 4;  // Q, Q^T, dO, dO^T tiles + lse, dlt rows
    constexpr int NC = HD / FE<T>::KC;
    constexpr int NQG = TR / FE<T>::KC / WG;  // q chunks per group and tile
    constexpr int MBG = 4 / WG;               // 16-query blocks per group and tile
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, grp = group_of(tid >> 6);
    const int ql = lane & 15, g = lane >> 4;
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        hd{p.heads, p.do_bs, p.do_hs, p.do_rs};
    const T *Q = (const T *)p.Q + hq.base(bh);
    const T *K = (const T *)p.K + hk.base(bh);
    const T *V = (const T *)p.V + hk.base(bh);
    const T *dO = (const T *)p.dO + hd.base(bh);
    const float *lse = p.lse + bh * p.sq, *dlt = p.dlt + bh * p.sq;
    const int key = kb * TR + wave * 16 + ql;  // this lane's key (column of S = Q.K^T)
    const bool kok = key < p.skv;
    const float c2 = p.scale * LOG2E;

    u32x4 kf[NC], vf[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const int64_t off = kok ? (int64_t)key * p.kv_rs + c * FE<T>::KC + g * FE<T>::VEC : 0;
        const u32x4 a = ld16(K + off), b = ld16(V + off);
        kf[c] = kok ? a : u32x4{0u, 0u, 0u, 0u};
        vf[c] = kok ? b : u32x4{0u, 0u, 0u, 0u};
    }
    f32x4 dk[4], dv[4];
#pragma unroll
    for (int n = 0; n < 4; ++n) dk[n] = dv[n] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int qblocks = (p.sq + TR - 1) / TR;
    const int qb0 = p.causal ? kb : 0;
    // Q and dO, each needed row-major (S, dP) and transposed (dK, dV); the rows' LSE (as log2) and
    // rowsum(dO * O) ride along.
    TilePair<T, NTH * WG> tp;
    tp.tid = tid;
    tp.m[0] = Q;
    tp.m[1] = dO;
    tp.rs[0] = p.q_rs;
    tp.rs[1] = p.do_rs;
    tp.rows[0] = tp.rows[1] = (int)p.sq;
    tp.off_rows[0] = 0;
    tp.off_cols[0] = T_;
    tp.off_rows[1] = 2 * T_;
    tp.off_cols[1] = 3 * T_;
    tp.aux[0] = lse;
    tp.aux[1] = dlt;
    tp.aux_scale[0] = LOG2E;
    tp.aux_off = 4 * T_;
    tp.aux_rows = (int)p.sq;
    pipelined(tp, smem, STAGE, qb0, qblocks - qb0, [&](int t, const char *st) {
        const int qb = qb0 + t;
        const char *qt = st, *qtt = st + T_, *dot = st + 2 * T_, *dott = st + 3 * T_;
        const float *ls = (const float *)(st + 4 * T_), *dl = ls + TR;
        // S = Q.K^T and dP = dO.V^T: rows q = 16mb + 4g + r of the tile (mb = grp * MBG + i),
        // column = this key.
        f32x4 sp[MBG], dp[MBG];
#pragma unroll
        for (int i = 0; i < MBG; ++i) {
            const int mb = grp * MBG + i;
            sp[i] = dp[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                mma16<T>(sp[i], frag_c<T>(qt, mb * 16 + ql, c, g), kf[c]);
                mma16<T>(dp[i], frag_c<T>(dot, mb * 16 + ql, c, g), vf[c]);
            }
        }
        // P = exp2(S * scale * log2(e) - LSE2). Rows past seq_q need no mask: their Q and dO rows
        // load as zeros (and their LSE as 0), so they add nothing. A key past seq_kv only reaches
        // its own dK, dV row, which is not stored. Only the causal diagonal block masks keys above
        // the query.
        // The mask sets the score to -inf (exp2(-inf) = 0) in a wave-uniform branch, so the other
        // blocks run the exponentials without a compare and select per probability.
        if (p.causal && qb == kb) {
#pragma unroll
            for (int i = 0; i < MBG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r)
                    if (key > qb * TR + (grp * MBG + i) * 16 + g * 4 + r) sp[i][r] = -INFINITY;
        }
#pragma unroll
        for (int i = 0; i < MBG; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int ql_ = (grp * MBG + i) * 16 + g * 4 + r;
                const float pr = exp2_fast(sp[i][r] * c2 - ls[ql_]);
                sp[i][r] = pr;
                dp[i][r] = pr * (dp[i][r] - dl[ql_]);
            }
        // dV (keys x d) += P^T (keys x q) . dO (q x d);  dK += dS^T . Q, over this group's queries
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int c = 0; c < NQG; ++c) {
                mma16<T>(dv[n], frag_acc<T>(sp, c), frag_s<T>(dott, n * 16 + ql, grp * NQG + c, g));
                mma16<T>(dk[n], frag_acc<T>(dp, c), frag_s<T>(qtt, n * 16 + ql, grp * NQG + c, g));
            }
    });
    if constexpr (WG == 2) {
        float v[32];
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                v[n * 4 + r] = dk[n][r];
                v[16 + n * 4 + r] = dv[n][r];
            }
        if (!hand_over<32>(smem, grp, wave, lane, v)) return;
#pragma unroll
        for (int n = 0; n < 4; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                dk[n][r] += v[n * 4 + r];
                dv[n][r] += v[16 + n * 4 + r];
            }
    }
    // Lane l holds rows (keys) 16*wave + 4g + r and column d = 16n + l%16.
    const Head hdk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs};
    float *dK = (float *)p.dK + hdk.base(bh), *dV = (float *)p.dV + hdk.base(bh);
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        const int k = kb * TR + wave * 16 + g * 4 + r;
        if (k >= p.skv) continue;
#pragma unroll
        for (int n = 0; n < 4; ++n) {
            dK[(int64_t)k * p.kv_rs + n * 16 + ql] = dk[n][r] * p.scale;
            dV[(int64_t)k * p.kv_rs + n * 16 + ql] = dv[n][r];
        }
    }
}


// dQ for 64 queries per block (16 per wave), looping over the key blocks they see. WG = 2: each
// wave group takes half of every key tile's rows (see flash_fwd).
template <typename T>
constexpr int dq_lds() { return 2 * 3 * tile_bytes<T>(); }

template <typename T, int WG>
__device__ __forceinline__ void dq_block(const FlashArgs &p, int qb, int64_t bh, char *smem) {
    constexpr int T_ = tile_bytes<T>();
    constexpr int STAGE = 3 * T_;  // K, V, K^T
    constexpr int NC = HD / FE<T>::KC;
    constexpr int NKG = TR / FE<T>::KC / WG;  // key chunks per group and tile
    constexpr int MBG = 4 / WG;               // 16-key blocks per group and tile
    const int tid = threadIdx.x, lane = tid & 63, wave = (tid >> 6) & 3, grp = group_of(tid >> 6);
    const int ql = lane & 15, g = lane >> 4;
    const Head hq{p.heads, p.q_bs, p.q_hs, p.q_rs}, hk{p.heads, p.kv_bs, p.kv_hs, p.kv_rs},
        hd{p.heads, p.do_bs, p.do_hs, p.do_rs};
    const T *Q = (const T *)p.Q + hq.base(bh);
    const T *K = (const T *)p.K + hk.base(bh);
    const T *V = (const T *)p.V + hk.base(bh);
    const T *dO = (const T *)p.dO + hd.base(bh);
    const int q = qb * TR + wave * 16 + ql;
    const bool qok = q < p.sq;
    const float c2 = p.scale * LOG2E;
    const float lse2 = qok ? p.lse[bh * p.sq + q] * LOG2E : 0.f;

    u32x4 qf[NC], of[NC];
#pragma unroll
    for (int c = 0; c < NC; ++c) {
        const u32x4 a = ld16(Q + (qok ? (int64_t)q * p.q_rs + c * FE<T>::KC + g * FE<T>::VEC : 0));
        const u32x4 b = ld16(dO + (qok ? (int64_t)q * p.do_rs + c * FE<T>::KC + g * FE<T>::VEC : 0));
        qf[c] = qok ? a : u32x4{0u, 0u, 0u, 0u};
        of[c] = qok ? b : u32x4{0u, 0u, 0u, 0u};
    }
    // rowsum(dO * O) of this query, written by flash_bwd_dlt.
    const float dl = qok ? p.dlt[bh * p.sq + q] : 0.f;
    f32x4 dq[4];
#pragma unroll
    for (int d = 0; d < 4; ++d) dq[d] = f32x4{0.f, 0.f, 0.f, 0.f};

    const int kblocks = (p.skv + TR - 1) / TR;
    const int nkb = p.causal ? min(kblocks, qb + 1) : kblocks;
    // K row-major (S^T) and transposed (dQ^T), V row-major (dP^T).
    TilePair<T, NTH * WG> tp;
    tp.tid = tid;
    tp.m[0] = K;
    tp.m[1] = V;
    tp.rs[0] = tp.rs[1] = p.kv_rs;
    tp.rows[0] = tp.rows[1] = (int)p.skv;
    tp.off_rows[0] = 0;
    tp.off_cols[0] = 2 * T_;
    tp.off_rows[1] = T_;
    tp.off_cols[1] = -1;
    pipelined(tp, smem, STAGE, 0, nkb, [&](int kb, const char *kt) {
        const char *vt = kt + T_, *ktt = kt + 2 * T_;
        // S^T = K.Q^T and dP^T = V.dO^T: rows = keys 16mb + 4g + r (mb = grp * MBG + i), column =
        // this query.
        f32x4 sp[MBG], dp[MBG];
#pragma unroll
        for (int i = 0; i < MBG; ++i) {
            const int mb = grp * MBG + i;
            sp[i] = dp[i] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int c = 0; c < NC; ++c) {
                mma16<T>(sp[i], frag_c<T>(kt, mb * 16 + ql, c, g), qf[c]);
                mma16<T>(dp[i], frag_c<T>(vt, mb * 16 + ql, c, g), of[c]);
            }
        }
        // Queries past seq_q are not stored. The causal diagonal block masks keys above the query,
        // and the last block keys past seq_kv (their K rows are zero, but an unmasked probability
        // exp2(-LSE2) could overflow and turn 0 * inf into NaN).
        // The masks set the score to -inf (exp2(-inf) = 0) in a wave-uniform branch that only these
        // blocks take.
        if ((p.causal && kb == qb) || (kb == nkb - 1 && p.skv % TR != 0)) {
#pragma unroll
            for (int i = 0; i < MBG; ++i)
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const int key = kb * TR + (grp * MBG + i) * 16 + g * 4 + r;
                    if (key >= p.skv || (p.causal && key > q)) sp[i][r] = -INFINITY;
                }
        }
#pragma unroll
        for (int i = 0; i < MBG; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) dp[i][r] = exp2_fast(sp[i][r] * c2 - lse2) * (dp[i][r] - dl);
        // dQ^T (d x q) += K^T (d x keys) . dS^T (keys x q), over this group's keys
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int c = 0; c < NKG; ++c)
                mma16<T>(dq[d], frag_s<T>(ktt, d * 16 + ql, grp * NKG + c, g), frag_acc<T>(dp, c));
    });
    if constexpr (WG == 2) {
        float v[16];
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[d * 4 + r] = dq[d][r];
        if (!hand_over<16>(smem, grp, wave, lane, v)) return;
#pragma unroll
        for (int d = 0; d < 4; ++d)
#pragma unroll
            for (int r = 0; r < 4; ++r) dq[d][r] += v[d * 4 + r];
    }
    if (qok) {
        float *dQ = (float *)p.dQ + hq.base(bh) + (int64_t)q * p.q_rs;
#pragma unroll
        for (int d = 0; d < 4; ++d) *(f32x4 *)(dQ + d * 16 + g * 4) = dq[d] * p.scale;
    }
}


// rowsum(dO * O) of every query row into p.dlt, 8 lanes per row (8 columns each), for
// flash_bwd_fused, whose dK/dV part reads rows that other blocks' dQ parts cover.
template <typename T>
__global__ __launch_bounds__(256) void flash_bwd_dlt(const FlashArgs p) {
    const int64_t row = (int64_t)blockIdx.x * 32 + (threadIdx.x >> 3);
    const int c = threadIdx.x & 7;
    if (row >= p.bh * p.sq) return;  // whole 8-lane groups leave together
    const int64_t bh = row / p.sq, q = row % p.sq;
    const Head hd{p.heads, p.do_bs, p.do_hs, p.do_rs}, ho{p.heads, p.o_bs, p.o_hs, p.o_rs};
    const float *o = (const float *)p.O + ho.base(bh) + q * p.o_rs + 8 * c;
    const f32x4 o0 = *(const f32x4 *)o, o1 = *(const f32x4 *)(o + 4);
    f32x4 d0, d1;
    if constexpr (sizeof(T) == 4) {
        const float *d = (const float *)p.dO + hd.base(bh) + q * p.do_rs + 8 * c;
        d0 = *(const f32x4 *)d;
        d1 = *(const f32x4 *)(d + 4);
    } else {
        const u32x4 h = *(const u32x4 *)((const uint16_t *)p.dO + hd.base(bh) + q * p.do_rs + 8 * c);
        d0 = f32x4{__uint_as_float(h[0] << 16), __uint_as_float(h[0] & 0xffff0000u), __uint_as_float(h[1] << 16),
                   __uint_as_float(h[1] & 0xffff0000u)};
        d1 = f32x4{__uint_as_float(h[2] << 16), __uint_as_float(h[2] & 0xffff0000u), __uint_as_float(h[3] << 16),
                   __uint_as_float(h[3] & 0xffff0000u)};
    }
    float s = d0[0] * o0[0] + d0[1] * o0[1] + d0[2] * o0[2] + d0[3] * o0[3] + d1[0] * o1[0] + d1[1] * o1[1] +
              d1[2] * o1[2] + d1[3] * o1[3];
#pragma unroll
    for (int w = 1; w < 8; w <<= 1) s += __shfl_xor(s, w, 64);
    if (c == 0) p.dlt[bh * p.sq + q] = s;
}

// The backward for grids with as many key blocks as query blocks: block j computes dQ of query
// block j, then dK and dV of key block j. Under the causal mask the two parts' tile counts are
// j + 1 and blocks - j, so every block does the same work (one kernel of balanced blocks in place
// of two kernels whose slowest blocks each take every tile).
template <typename T, int WG>
__global__ __launch_bounds__(NTH * WG) void flash_bwd_fused(const FlashArgs p) {
    __shared__ __attribute__((aligned(16))) char smem[dkdv_lds<T>() > dq_lds<T>() ? dkdv_lds<T>() : dq_lds<T>()];
    const int j = (int)blockIdx.x;
    const int64_t bh = blockIdx.y;
    dq_block<T, WG>(p, j, bh, smem);
    __syncthreads();  // the dQ part's last LDS reads (its hand-over) before the dK/dV part's writes
    dkdv_block<T, WG>(p, j, bh, smem);
}

}  // namespace

bool flash_supported(const FlashArgs &p, int elem_bytes, bool backward) {
    const int64_t vec = 16 / elem_bytes;
    auto ok = [&](const void *ptr, int64_t bs, int64_t hs, int64_t rs, int64_t v) {
        return ptr && (uintptr_t)ptr % 16 == 0 && bs % v == 0 && hs % v == 0 && rs % v == 0;
    };
    bool r = p.head_dim == HD && ok(p.Q, p.q_bs, p.q_hs, p.q_rs, vec) && ok(p.K, p.kv_bs, p.kv_hs, p.kv_rs, vec) &&
             ok(p.V, p.kv_bs, p.kv_hs, p.kv_rs, vec);
    if (backward)
        r = r && ok(p.dO, p.do_bs, p.do_hs, p.do_rs, vec) && ok(p.dQ, p.q_bs, p.q_hs, p.q_rs, 4) &&
            ok(p.dK, p.kv_bs, p.kv_hs, p.kv_rs, 4) && ok(p.dV, p.kv_bs, p.kv_hs, p.kv_rs, 4);
    else
        r = r && ok(p.O, p.o_bs, p.o_hs, p.o_rs, 4);
    return r;
}

// Grids of at most this many blocks (one round on MI355X's 256 CUs) run the two-group form: with
// one block per CU, each of a block's 16-row jobs then runs as two waves.
constexpr int64_t SPLIT_MAX_BLOCKS = 256;

template <typename T, int WG>
void fwd_launch(hipStream_t s, const FlashArgs &p, dim3 grid) {
    hipLaunchKernelGGL((flash_fwd<T, WG>), grid, dim3(NTH * WG), 0, s, p);
}

template <typename T, int WG>
void bwd_launch(hipStream_t s, const FlashArgs &p, int64_t blocks) {
    // rowsum(dO * O) for every row first, then one kernel of balanced dQ + dK/dV blocks.
    const int64_t rows = p.bh * p.sq;
    hipLaunchKernelGGL(flash_bwd_dlt<T>, dim3((unsigned)((rows + 31) / 32)), dim3(256), 0, s, p);
    hipLaunchKernelGGL((flash_bwd_fused<T, WG>), dim3((unsigned)blocks, (unsigned)p.bh), dim3(NTH * WG), 0, s, p);
}

it_status launch_flash_fwd(hipStream_t s, const FlashArgs &p, bool bf16) {
    if (bf16 && flash2_applicable(p, false)) return launch_flash2_fwd(s, p);
    if (p.o_bf16) return fail(IT_ERR_DIMS, "flash attention: a BF16 O needs the BF16 kernels' 2 GiB row limits");
    const int64_t qblocks = (p.sq + TR - 1) / TR;
    if (qblocks > 0x7fffffff || p.bh > 65535) return fail(IT_ERR_DIMS, "flash attention: grid too large");
    const dim3 grid((unsigned)qblocks, (unsigned)p.bh);
    const bool split = qblocks * p.bh <= SPLIT_MAX_BLOCKS;
    if (bf16)
        split ? fwd_launch<uint16_t, 2>(s, p, grid) : fwd_launch<uint16_t, 1>(s, p, grid);
    else
        split ? fwd_launch<float, 2>(s, p, grid) : fwd_launch<float, 1>(s, p, grid);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_flash_bwd(hipStream_t s, const FlashArgs &p, bool bf16) {
    // The backward entry points take one sequence length for queries and keys.
    if (p.sq != p.skv) return fail(IT_ERR_SHAPE, "flash attention backward: query and key lengths differ");
    if (bf16 && flash2_applicable(p, true)) return launch_flash2_bwd(s, p);
    if (p.o_bf16 || p.grad_bf16)
        return fail(IT_ERR_DIMS, "flash attention backward: BF16 O or gradients need the BF16 kernels' 2 GiB row limits");
    const int64_t blocks = (p.sq + TR - 1) / TR;
    if (blocks > 0x7fffffff || p.bh > 65535) return fail(IT_ERR_DIMS, "flash attention backward: grid too large");
    const bool split = blocks * p.bh <= SPLIT_MAX_BLOCKS;
    if (bf16)
        split ? bwd_launch<uint16_t, 2>(s, p, blocks) : bwd_launch<uint16_t, 1>(s, p, blocks);
    else
        split ? bwd_launch<float, 2>(s, p, blocks) : bwd_launch<float, 1>(s, p, blocks);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

}  // namespace it
