// MFMA GEMM kernels for gfx950 (CDNA4): FP32 (v_mfma_f32_16x16x4_f32) and BF16-in / FP32-accumulate
// (v_mfma_f32_16x16x32_bf16), with the transposed-operand variant chosen at launch, strided and
// two-level batching, split-K with a deterministic reduction, and fused epilogues (alpha/beta,
// bias, SwiGLU dual-B, causal mask).
//
// Replaces the Metal GEMMs gemm_f32/_tiled/_batched (src/shaders/gemm.metal:15-119), the backward
// gemm_grad_a/_b and batched forms (src/shaders/backward/gemm.metal:20-120), the BF16 GEMMs
// (src/shaders/bf16_ops.metal:25-122) and the closed MPSMatrixMultiplication calls
// (src/ops/mps_gemm.rs:169-198,278-306,390-418,519-553).
//
// Design (per 256-thread workgroup = 4 wave64s):
//   * Block tile BM x BN, k-tile BK = 128 bytes of one operand row (32 f32 or 64 bf16).
//   * Operands whose global layout is k-contiguous are copied global -> LDS with 128-bit loads and
//     stores into a [rows][BK] tile with a 144-byte pitch; a lane's MFMA fragment is then one
//     128-bit LDS read (16 lanes on 16 rows at one k offset hit disjoint banks with that pitch).
//   * mn-contiguous operands (A stored [K,M], B stored [K,N]): FP32 keeps the [k][mn] tile and reads
//     its fragment as four 32-bit LDS loads; BF16 transposes 4 k-rows x 8 columns in registers on
//     the way into LDS so the fragment stays a single 128-bit read. No transpose is ever
//     materialised in HBM.
//   * Two LDS stages: global loads of tile t+1 are in flight while tile t is multiplied; one
//     barrier per k-tile.
//   * A lane's fragment covers k = 4g..4g+3 (FP32) or 8g..8g+7 (BF16) of a 16/32-wide k step, where
//     g = lane / 16. A and B use the same k assignment, so every MFMA sums the right products; the
//     summation order differs from a sequential loop only by FP32 rounding.
//   * Tiles are enumerated XCD-aware: the 8 XCDs each receive a contiguous range of the grouped
//     tile order, so blocks sharing A rows or B columns hit the same L2.
#include <cmath>
#include <cstdlib>
#include <cstdio>
#include <string>
#include <type_traits>

#include "epilogue.hpp"
#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

constexpr int NTHREADS = 256;
constexpr int ROW_PITCH = 144;  // LDS bytes per row of a [rows][BK] tile (128 data + 16 pad)

template <typename T>
struct ET;
template <>
struct ET<float> {
    static constexpr int VEC = 4;    // elements per 16 bytes
    static constexpr int BK = 32;    // k per tile
    static constexpr int KSTEP = 16; // k per fragment step (4 lane groups x 4)
};
template <>
struct ET<uint16_t> {
    static constexpr int VEC = 8;
    static constexpr int BK = 64;
    static constexpr int KSTEP = 32;
};


// Loads VEC consecutive elements starting at base[off]; elements at positions c + e >= clim (or the
// whole vector when !row_ok) read as zero.
template <typename T>
__device__ __forceinline__ u32x4 load_vec(const T *base, int64_t off, bool row_ok, int64_t c,
                                          int64_t clim, bool vec_ok) {
    constexpr int VEC = ET<T>::VEC;
    if (row_ok && vec_ok && c + VEC <= clim) return *(const u32x4 *)(base + off);
    u32x4 v = {0u, 0u, 0u, 0u};
    if (row_ok) {
        if constexpr (sizeof(T) == 4) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (c + e < clim) v[e] = __float_as_uint(base[off + e]);
        } else {
#pragma unroll
            for (int e = 0; e < 8; ++e)
                if (c + e < clim) v[e >> 1] |= (uint32_t)base[off + e] << ((e & 1) * 16);
        }
    }
    return v;
}

// How an operand tile is read from global memory:
//   LOAD_EXACT   every tile is whole and aligned: plain 128-bit loads;
//   LOAD_MASKED  16-byte vectors are aligned and never straddle an edge, so a vector is either
//                wholly in bounds or wholly out: branch-free load of a safe address + select;
//   LOAD_CHECKED anything else: per-element bounds checks.
//   LOAD_RSRC    (FP32, 16-byte vectors as LOAD_MASKED, K a multiple of the k-tile where an operand
//                is k-contiguous) buffer loads through a descriptor that ends where the operand's
//                valid rows (k-contiguous) or k (mn-contiguous) end, from 32-bit offsets formed once
//                per block: the hardware's range check returns zeros past that end, with no
//                per-load address arithmetic or selects. The descriptor spans exactly the
//                operand's elements (first to last, not whole row strides, which can reach past the
//                allocation for a strided head). An mn-contiguous operand's columns past M (or N)
//                read the next row's elements, or zeros past the last element; they reach only
//                output rows (columns) past M (N), which the epilogue never stores.
enum LoadMode : int { LOAD_EXACT = 0, LOAD_MASKED = 1, LOAD_CHECKED = 2, LOAD_RSRC = 3 };

template <int MODE, typename T>
__device__ __forceinline__ u32x4 load_mode(const T *base, int64_t off, bool row_ok, int64_t c,
                                           int64_t clim, bool vec_ok) {
    if constexpr (MODE == LOAD_EXACT) {
        return *(const u32x4 *)(base + off);
    } else if constexpr (MODE == LOAD_MASKED) {
        const bool ok = row_ok && c < clim;
        const u32x4 v = *(const u32x4 *)(base + (ok ? off : 0));
        return ok ? v : u32x4{0u, 0u, 0u, 0u};
    } else {
        return load_vec<T>(base, off, row_ok, c, clim, vec_ok);
    }
}

// One operand's k-tile: global -> registers -> LDS, and LDS -> MFMA fragments.
//   KCONTIG: global element (r, k) at base[r * ld + k] (A not transposed, or B transposed).
//   otherwise: global element (r, k) at base[k * ld + r].
template <typename T, bool KCONTIG, int ROWS>
struct Operand {
    static constexpr int VEC = ET<T>::VEC;
    static constexpr int BK = ET<T>::BK;
    static constexpr bool TRANSPOSE = !KCONTIG && sizeof(T) == 2;  // bf16 [k][mn] -> LDS [mn][k]
    static constexpr bool KMAJOR_LDS = !KCONTIG && sizeof(T) == 4;  // f32 keeps [k][mn] in LDS
    static constexpr int KMAJOR_PITCH = ROWS * 4 + 16;
    static constexpr int STAGE_BYTES = KMAJOR_LDS ? BK * KMAJOR_PITCH : ROWS * ROW_PITCH;
    static constexpr int ITEMS = TRANSPOSE ? (BK / 4) * (ROWS / VEC) : ROWS * BK / VEC;
    static constexpr int LOADS = TRANSPOSE ? 4 : 1;
    static constexpr int ITERS = (ITEMS + NTHREADS - 1) / NTHREADS;
    static constexpr int KGROUPS = BK / 4;

    u32x4 reg[ITERS][LOADS];

    // Transposed units are (k-group of 4 rows, 8 columns). Lane bit 0 picks one of two adjacent
    // column chunks and bits 1..4 the k-group, so the 8-byte LDS stores of 32 consecutive lanes
    // land in 64 distinct banks (two rows 8 apart, 16 k offsets each).
    __device__ __forceinline__ static void unit(int item, int &kg, int &rc) {
        rc = (item & 1) | ((item / (2 * KGROUPS)) << 1);
        kg = (item >> 1) % KGROUPS;
    }

    template <int MODE = LOAD_CHECKED>
    __device__ __forceinline__ void load(const T *base, int64_t ld, int64_t r0, int64_t k0,
                                         int64_t rlim, int64_t klim, bool vec_ok, int tid) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
            if constexpr (KCONTIG) {
                const int rr = item / (BK / VEC), kc = item % (BK / VEC);
                const int64_t gr = r0 + rr, gk = k0 + kc * VEC;
                reg[it][0] = load_mode<MODE>(base, gr * ld + gk, gr < rlim, gk, klim, vec_ok);
            } else if constexpr (!TRANSPOSE) {
                const int kk = item / (ROWS / VEC), rc = item % (ROWS / VEC);
                const int64_t gk = k0 + kk, gr = r0 + rc * VEC;
                reg[it][0] = load_mode<MODE>(base, gk * ld + gr, gk < klim, gr, rlim, vec_ok);
            } else {
                int kg, rc;
                unit(item, kg, rc);
                const int64_t gr = r0 + rc * VEC;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int64_t gk = k0 + kg * 4 + q;
                    reg[it][q] = load_mode<MODE>(base, gk * ld + gr, gk < klim, gr, rlim, vec_ok);
                }
            }
        }
    }

    // Per-k scale of a k-contiguous FP32 tile (the RMSNorm gamma of a fused norm + projection):
    // load_kscale fetches s[k] for this thread's elements with the tile's own loads, apply_kscale
    // multiplies the loaded elements before they go to LDS (elements at k >= klim are zeros).
    f32x4 kscale[ITERS];

    __device__ __forceinline__ void load_kscale(const float *s, int64_t k0, int64_t klim, int tid) {
        static_assert(KCONTIG && sizeof(T) == 4, "k scaling applies to k-contiguous FP32 tiles");
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
            const int64_t gk = k0 + (item % (BK / VEC)) * VEC;
            if (gk + 4 <= klim && (uintptr_t)(s + gk) % 16 == 0) {
                kscale[it] = *(const f32x4 *)(s + gk);
            } else {
#pragma unroll
                for (int e = 0; e < 4; ++e) kscale[it][e] = gk + e < klim ? s[gk + e] : 0.f;
            }
        }
    }

    // Adds the squares of this thread's loaded elements to ss[it] (the rows of a thread's items are
    // the same in every k-tile).
    __device__ __forceinline__ void add_squares(float (&ss)[ITERS], int tid) const {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float v = __uint_as_float(reg[it][0][e]);
                ss[it] += v * v;
            }
        }
    }

    __device__ __forceinline__ void apply_kscale(int tid) {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
#pragma unroll
            for (int e = 0; e < 4; ++e)
                reg[it][0][e] = __float_as_uint(__uint_as_float(reg[it][0][e]) * kscale[it][e]);
        }
    }

    // Softmax cross-entropy gradient of FP32 logits (the A operand of dL/dh = G.E or dL/dE =
    // G^T.h): load_xent fetches, with the tile, each item's token statistics {max, 1/sum} and
    // target (rows are tokens when k-contiguous, k is the token otherwise); apply_xent turns the
    // loaded logits into (exp(x - max) / sum - onehot) * scale, and elements outside the product
    // (tokens or classes past the limits) into zeros.
    float2 xs[ITERS];
    uint32_t xt[ITERS];
    int64_t xk0;

    __device__ __forceinline__ void load_xent(const float2 *st, const uint32_t *tg, int64_t r0, int64_t k0,
                                              int64_t rlim, int64_t klim, int tid) {
        static_assert(sizeof(T) == 4, "cross-entropy gradients are FP32");
        xk0 = k0;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
            const int64_t tok = KCONTIG ? r0 + item / (BK / VEC) : k0 + item / (ROWS / VEC);
            const bool ok = tok < (KCONTIG ? rlim : klim);
            xs[it] = ok ? st[tok] : float2{INFINITY, 0.f};
            xt[it] = ok ? tg[tok] : 0xffffffffu;
        }
    }

    // exp(x - max) as 2^((x - max) log2 e) on the hardware unit: a few VALU operations per element,
    // since every element of the A tile goes through it (relative error about 1e-6 for a logit 20
    // below the row max, where the probability itself is below 1e-8).
    template <bool CHECK>
    __device__ __forceinline__ void apply_xent(int64_t r0, int64_t rlim, int64_t klim, float scale, int tid) {
        constexpr float LOG2E = 1.4426950408889634f;
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
            const int64_t c0 = KCONTIG ? xk0 + (item % (BK / VEC)) * VEC : r0 + (item % (ROWS / VEC)) * VEC;
            const int64_t clim = KCONTIG ? klim : rlim;
            const float mx = xs[it].x, ps = xs[it].y * scale;
            const int32_t tc = (int32_t)(xt[it] - (uint32_t)c0);  // target's offset in this vector
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                const float x = __uint_as_float(reg[it][0][e]);
                float g = __builtin_amdgcn_exp2f((x - mx) * LOG2E) * ps - (tc == e ? scale : 0.f);
                if constexpr (CHECK) g = c0 + e < clim ? g : 0.f;
                reg[it][0][e] = __float_as_uint(g);
            }
        }
    }

    __device__ __forceinline__ void store(char *lds, int tid) const {
#pragma unroll
        for (int it = 0; it < ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (ITEMS % NTHREADS != 0 && item >= ITEMS) continue;
            if constexpr (KCONTIG) {
                const int rr = item / (BK / VEC), kc = item % (BK / VEC);
                *(u32x4 *)(lds + rr * ROW_PITCH + kc * 16) = reg[it][0];
            } else if constexpr (!TRANSPOSE) {
                const int kk = item / (ROWS / VEC), rc = item % (ROWS / VEC);
                *(u32x4 *)(lds + kk * KMAJOR_PITCH + rc * 16) = reg[it][0];
            } else {
                int kg, rc;
                unit(item, kg, rc);
                const u32x4 &v0 = reg[it][0], &v1 = reg[it][1], &v2 = reg[it][2], &v3 = reg[it][3];
#pragma unroll
                for (int d = 0; d < 4; ++d) {
                    // columns 2d (low halves) and 2d+1 (high halves) of the 4 loaded k-rows
                    u32x2 lo, hi;
                    lo[0] = (v0[d] & 0xffffu) | (v1[d] << 16);
                    lo[1] = (v2[d] & 0xffffu) | (v3[d] << 16);
                    hi[0] = (v0[d] >> 16) | (v1[d] & 0xffff0000u);
                    hi[1] = (v2[d] >> 16) | (v3[d] & 0xffff0000u);
                    *(u32x2 *)(lds + (rc * 8 + 2 * d) * ROW_PITCH + kg * 8) = lo;
                    *(u32x2 *)(lds + (rc * 8 + 2 * d + 1) * ROW_PITCH + kg * 8) = hi;
                }
            }
        }
    }

    // v_mfma_f32_32x32x16_bf16 fragment: lane l supplies row `row + l % 32` and the 8 k values
    // 8*(l/32)..8*(l/32)+7 of the 16-wide k step `ks` (bf16 tiles in [rows][BK] layout only).
    __device__ __forceinline__ static u32x4 frag32(const char *lds, int row, int ks, int lane) {
        return *(const u32x4 *)(lds + (row + (lane & 31)) * ROW_PITCH + ks * 32 + (lane >> 5) * 16);
    }

    // Fragment of the 16 rows starting at `row` for fragment step `ks`.
    __device__ __forceinline__ static u32x4 frag(const char *lds, int row, int ks, int lane) {
        const int i = lane & 15, g = lane >> 4;
        if constexpr (!KMAJOR_LDS) {
            return *(const u32x4 *)(lds + (row + i) * ROW_PITCH + ks * 64 + g * 16);
        } else {
            u32x4 v;
            const int k = ks * 16 + g * 4;
#pragma unroll
            for (int s = 0; s < 4; ++s) v[s] = *(const uint32_t *)(lds + (k + s) * KMAJOR_PITCH + (row + i) * 4);
            return v;
        }
    }
};

// LOAD_RSRC addressing of one FP32 operand tile (Operand<float, KCONTIG, ROWS>'s items): the
// descriptor and each item's byte offset at k-tile 0; a k-tile adds k0 * kstride bytes.
template <bool KCONTIG, int ROWS>
struct RsrcLoad {
    using O = Operand<float, KCONTIG, ROWS>;
    __amdgpu_buffer_rsrc_t rs;
    uint32_t voff[O::ITERS];
    uint32_t kstride;

    // base: the operand of this batch item; records: its extent in bytes, ((rows - 1) * ld + K) * 4
    // k-contiguous, ((K - 1) * ld + rows) * 4 otherwise (exactly the operand's span: a row stride past
    // the last element may leave the allocation); r0: the tile's first row.
    __device__ __forceinline__ void init(const float *base, int64_t ld, int64_t r0, int64_t records, int tid) {
        const int n = records > 0x7fffffff ? 0x7fffffff : (int)records;
        rs = __builtin_amdgcn_make_buffer_rsrc(const_cast<float *>(base), (short)0, n, 0x00020000);
        kstride = KCONTIG ? 4u : (uint32_t)(ld * 4);
#pragma unroll
        for (int it = 0; it < O::ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if constexpr (KCONTIG) {
                const int rr = item / (O::BK / O::VEC), kc = item % (O::BK / O::VEC);
                voff[it] = (uint32_t)(((r0 + rr) * ld + kc * O::VEC) * 4);
            } else {
                const int kk = item / (ROWS / O::VEC), rc = item % (ROWS / O::VEC);
                voff[it] = (uint32_t)((kk * ld + r0 + rc * O::VEC) * 4);
            }
        }
    }

    __device__ __forceinline__ void load(O &o, int64_t k0, int tid) const {
        const uint32_t koff = (uint32_t)k0 * kstride;
#pragma unroll
        for (int it = 0; it < O::ITERS; ++it) {
            const int item = tid + it * NTHREADS;
            if (O::ITEMS % NTHREADS != 0 && item >= O::ITEMS) continue;
            o.reg[it][0] = __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, voff[it] + koff, 0, 0));
        }
    }
};

template <typename T>
__device__ __forceinline__ void mma(f32x4 &acc, const u32x4 &a, const u32x4 &b) {
    if constexpr (sizeof(T) == 4) {
#pragma unroll
        for (int s = 0; s < 4; ++s)
            acc = __builtin_amdgcn_mfma_f32_16x16x4f32(__uint_as_float(a[s]), __uint_as_float(b[s]),
                                                       acc, 0, 0, 0);
    } else {
        acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                      __builtin_bit_cast(bf16x8, b), acc, 0, 0, 0);
    }
}

// Grouped raster order: tile `idx` of groups of 8 tile rows, column-major within a group.
__device__ __forceinline__ void raster_tile(int idx, int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int GROUP = 8;
    const int span = GROUP * tiles_n;
    const int first_m = (idx / span) * GROUP;
    const int gsize = min(tiles_m - first_m, GROUP);
    const int in = idx % span;
    tm = first_m + in % gsize;
    tn = in / gsize;
}

// Tile order: XCD-aware remap (workgroup w runs on XCD w % 8, which then takes a contiguous range
// of the grouped order) then the grouped raster.
__device__ __forceinline__ void map_tile(int pid, int tiles_m, int tiles_n, int &tm, int &tn) {
    constexpr int NXCD = 8;
    const int total = tiles_m * tiles_n;
    if (total % NXCD == 0) pid = (pid % NXCD) * (total / NXCD) + pid / NXCD;
    raster_tile(pid, tiles_m, tiles_n, tm, tn);
}

namespace sg {
constexpr int MFMA = 0x008, VMEM_READ = 0x020, DS_READ = 0x100, DS_WRITE = 0x200;
}

constexpr int CP_DEVICE_SCOPE = 16;  // cache-policy bit sc1 of the buffer intrinsics: device scope

// LDS bytes of one gemm_mfma block (two stages of the A and B tiles).
template <typename T, bool TA, bool TB, int BM, int BN>
constexpr int mfma_smem_bytes() {
    return 2 * (Operand<T, !TA, BM>::STAGE_BYTES + Operand<T, TB, BN>::STAGE_BYTES);
}

// One block of gemm_mfma: output tile `tile` (in map_tile order) of batch-and-split index z, with
// `smem` of mfma_smem_bytes().
// FIX (64 x 64 tiles of batch-1 products): with split K, each split's partial tile goes to p.partial
// at device scope and the tile's last block to arrive at `arrive` (a zero counter, left at zero)
// adds the splits in split order and runs the epilogue, so no separate reduction launch follows.
template <typename T, bool TA, bool TB, int BM, int BN, int WM, int WN, bool DUAL, int LM, bool KS = false, int PF = 1,
          bool XF = false, bool FIX = false>
__device__ __forceinline__ void gemm_mfma_block(const GemmArgs &p, int tile, int64_t z, char *smem,
                                                int *arrive = nullptr) {
    static_assert(WM * WN == 4, "4 waves per block");
    constexpr int BK = ET<T>::BK;
    constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 16, FN = WTN / 16;
    // 64x64 tiles store straight from transposed accumulators (measured 1-6% faster on the TINY
    // step's small GEMMs); 128x128 tiles keep the LDS-staged epilogue, whose full-line stores
    // measured 3.5% faster on the LM-head forward's 268 MB of logits; SwiGLU pairs waves in LDS.
    constexpr bool XPOSE = !DUAL && BM == 64;
    using OA = Operand<T, !TA, BM>;
    using OB = Operand<T, TB, BN>;
    using OBH = Operand<T, TB, BN / 2>;  // DUAL: gate and up halves of the B tile
    static_assert(!DUAL || (!TA && TB), "SwiGLU is Y = X.W^T");
    constexpr int SA = OA::STAGE_BYTES, SB = OB::STAGE_BYTES;
    constexpr int STAGE = SA + SB;

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WN, wn = wave % WN;
    int tm, tn;
    map_tile(tile, p.tiles_m, p.tiles_n, tm, tn);
    const int64_t b = z % p.batch, split = z / p.batch;
    const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
    const T *A = (const T *)p.A + bo * p.sA_out + bi * p.sA_in;
    const T *B = (const T *)p.B + bo * p.sB_out + bi * p.sB_in;
    const T *B2 = DUAL ? (const T *)p.B2 + bo * p.sB_out + bi * p.sB_in : nullptr;
    const int64_t coff = bo * p.sC_out + bi * p.sC_in;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (DUAL ? BN / 2 : BN);

    if (p.causal != CAUSAL_NONE && n0 > m0 + BM - 1 + p.causal_offset) {
        // Entire tile is above the diagonal: no products needed.
        if (p.causal == CAUSAL_WRITE) {
            for (int e = tid; e < BM * BN; e += NTHREADS) {
                const int64_t row = m0 + e / BN, col = n0 + e % BN;
                if (row < p.M && col < p.N) store_out(p.C, coff + row * p.ldc + col, -INFINITY, p.out_bf16);
            }
        }
        return;
    }

    int64_t kb = split * p.k_per_split;
    int64_t ke = min(p.K, kb + p.k_per_split);
    if (p.kmode == KMODE_LOWER) ke = min(ke, m0 + BM);
    if (p.kmode == KMODE_UPPER) kb = max(kb, (m0 / BK) * BK);
    const int ntiles = ke > kb ? (int)((ke - kb + BK - 1) / BK) : 0;

    f32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Register staging sets: PF of them, so the loads of tile t+PF are issued during tile t.
    OA oa[PF];
    constexpr bool RSRC = LM == LOAD_RSRC;
    static_assert(!RSRC || (sizeof(T) == 4 && !DUAL && !KS && !XF), "LOAD_RSRC: plain FP32 tiles");
    RsrcLoad<!TA, BM> ra;
    RsrcLoad<TB, BN> rb;
    if constexpr (RSRC) {
        ra.init((const float *)A, p.lda, m0, (TA ? (p.K - 1) * p.lda + p.M : (p.M - 1) * p.lda + p.K) * 4, tid);
        rb.init((const float *)B, p.ldb, n0, (TB ? (p.N - 1) * p.ldb + p.K : (p.K - 1) * p.ldb + p.N) * 4, tid);
    }
    // SwiGLU (DUAL): the B tile's rows 0..BN/2-1 are gate-weight rows and BN/2..BN-1 the same up-
    // weight rows, so waves wn = 0 / 1 accumulate gate / up of one BM x BN/2 output tile and the
    // loop is the ordinary one.
    std::conditional_t<DUAL, OBH, OB> ob[PF];
    std::conditional_t<DUAL, OBH, char> ob2[PF];
    auto gload = [&](int set, int64_t k0) {
#pragma unroll
        for (int q = 0; q < PF; ++q)
            if (q == set) {
                if constexpr (RSRC) {
                    ra.load(oa[q], k0, tid);
                    rb.load(ob[q], k0, tid);
                } else {
                    oa[q].template load<LM>(A, p.lda, m0, k0, p.M, ke, p.a_vec_ok, tid);
                    if constexpr (KS) oa[q].load_kscale(p.a_kscale, k0, ke, tid);
                    if constexpr (XF) oa[q].load_xent(p.xent_stats, p.xent_tgt, m0, k0, p.M, ke, tid);
                    ob[q].template load<LM>(B, p.ldb, n0, k0, p.N, ke, p.b_vec_ok, tid);
                    if constexpr (DUAL) ob2[q].template load<LM>(B2, p.ldb, n0, k0, p.N, ke, p.b_vec_ok, tid);
                }
            }
    };
    // KS: per-thread partial sums of squares of its A rows, over the k-tiles written to LDS.
    float ssq[KS ? OA::ITERS : 1];
#pragma unroll
    for (int i = 0; i < (KS ? OA::ITERS : 1); ++i) ssq[i] = 0.f;
    auto gstore = [&](int set, char *st, bool fresh = true) {
#pragma unroll
        for (int q = 0; q < PF; ++q)
            if (q == set) {
                if constexpr (KS) {
                    if (fresh) oa[q].add_squares(ssq, tid);
                    oa[q].apply_kscale(tid);
                }
                if constexpr (XF) oa[q].template apply_xent<LM != LOAD_EXACT>(m0, p.M, ke, p.xent_scale, tid);
                oa[q].store(st, tid);
                ob[q].store(st + SA, tid);
                if constexpr (DUAL) ob2[q].store(st + SA + OBH::STAGE_BYTES, tid);
            }
    };
    {
        // Software-pipelined loop: fragments of k-step 1 are read while the MFMAs of k-step 0
        // issue; tile t+PF's global loads go out with k-step 0 (into the register set tile t+1 is
        // not using) and tile t+1 lands in the other LDS stage during k-step 1; prefetches past the
        // last tile re-read it into a dead stage.
        if (ntiles > 0) {
            u32x4 fa0[FM], fb0[FN], fa1[FM], fb1[FN];
            const int last = ntiles - 1;
            auto frags = [&](u32x4 (&fa)[FM], u32x4 (&fb)[FN], const char *st, int ks) {
#pragma unroll
                for (int i = 0; i < FM; ++i) fa[i] = OA::frag(st, wm * WTM + i * 16, ks, lane);
#pragma unroll
                for (int j = 0; j < FN; ++j) fb[j] = OB::frag(st + SA, wn * WTN + j * 16, ks, lane);
            };
            auto mmas = [&](const u32x4 (&fa)[FM], const u32x4 (&fb)[FN]) {
#pragma unroll
                for (int i = 0; i < FM; ++i)
#pragma unroll
                    for (int j = 0; j < FN; ++j) {
                        // XPOSE: B as the MFMA's row operand, the block comes out transposed.
                        if constexpr (XPOSE)
                            mma<T>(acc[i][j], fb[j], fa[i]);
                        else
                            mma<T>(acc[i][j], fa[i], fb[j]);
                    }
            };
            static_assert(BK / ET<T>::KSTEP == 2, "two fragment steps per k-tile");
            constexpr int MF = FM * FN * (sizeof(T) == 4 ? 4 : 1);
            constexpr int DSR = FM * (OA::KMAJOR_LDS ? 4 : 1) + FN * (OB::KMAJOR_LDS ? 4 : 1);
            constexpr int VMR = OA::ITERS * OA::LOADS + OB::ITERS * OB::LOADS;
            constexpr int DSW = OA::ITERS * (OA::TRANSPOSE ? 8 : 1) + OB::ITERS * (OB::TRANSPOSE ? 8 : 1);
            constexpr int G = MF < 8 ? MF : 8;
            gload(0, kb);
            gstore(0, smem);
#pragma unroll
            for (int q = 1; q < PF; ++q) gload(q, kb + (int64_t)min(q, last) * BK);
            __syncthreads();
            frags(fa0, fb0, smem, 0);
            auto tile = [&](int t, int pf_set, int nx_set) {
                const char *cur = smem + (t & 1) * STAGE;
                char *nxt = smem + ((t + 1) & 1) * STAGE;
                const int64_t kp = kb + (int64_t)min(t + PF, last) * BK;
                frags(fa1, fb1, cur, 1);
                if (PF == 1) {
                    gload(pf_set, kp);
                    mmas(fa0, fb0);
                    gstore(nx_set, nxt, t + 1 < ntiles);
                } else {
                    mmas(fa0, fb0);
                    gstore(nx_set, nxt, t + 1 < ntiles);
                    gload(pf_set, kp);
                }
                mmas(fa1, fb1);
                if constexpr (LM != LOAD_CHECKED) {
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        __builtin_amdgcn_sched_group_barrier(sg::DS_READ, (DSR + G - 1) / G, 0);
                        __builtin_amdgcn_sched_group_barrier(sg::VMEM_READ, (VMR + G - 1) / G, 0);
                        __builtin_amdgcn_sched_group_barrier(sg::MFMA, MF / G, 0);
                    }
#pragma unroll
                    for (int g = 0; g < G; ++g) {
                        __builtin_amdgcn_sched_group_barrier(sg::DS_WRITE, (DSW + G - 1) / G, 0);
                        __builtin_amdgcn_sched_group_barrier(sg::MFMA, MF / G, 0);
                    }
                }
                __syncthreads();
                frags(fa0, fb0, nxt, 0);
            };
            if constexpr (PF == 1) {
                for (int t = 0; t < ntiles; ++t) tile(t, 0, 0);
            } else {
                // Tile u's registers are set u % PF: tile t writes set (t+1) % PF to LDS and
                // reloads set t % PF (written to LDS during tile t-1) with tile t+PF.
                // Whole groups of PF tiles in a branch-free body, then the remaining tiles.
                int t = 0;
                for (; t + PF <= ntiles; t += PF) {
#pragma unroll
                    for (int q = 0; q < PF; ++q) tile(t + q, q, (q + 1) % PF);
                }
#pragma unroll
                for (int q = 0; q + 1 < PF; ++q)
                    if (t + q < ntiles) tile(t + q, q, (q + 1) % PF);
            }
        }
    }

    // KS: row sums of squares -> 1/rms per block row (the 8 threads of a row are 8 consecutive lanes).
    __shared__ float row_inv[KS ? BM : 1];
    if constexpr (KS) {
        constexpr int PER_ROW = BK / ET<T>::VEC;
        static_assert(PER_ROW == 8 && NTHREADS % PER_ROW == 0, "row partials sit in 8 consecutive lanes");
#pragma unroll
        for (int it = 0; it < OA::ITERS; ++it) {
            float v = ssq[it];
#pragma unroll
            for (int o = 1; o < PER_ROW; o <<= 1) v += __shfl_xor(v, o, 64);
            const int item = tid + it * NTHREADS;
            if ((OA::ITEMS % NTHREADS == 0 || item < OA::ITEMS) && tid % PER_ROW == 0) {
                const float rms = sqrtf(v / (float)p.K + p.rms_eps);
                row_inv[item / PER_ROW] = 1.0f / rms;
            }
        }
    }

    static_assert(!FIX || (XPOSE && !KS && !XF), "the in-kernel split-K sum covers plain 64 x 64 tiles");
    if constexpr (FIX) {
        if (p.splits > 1) {
            // Partial tile of split z at device scope (written through this XCD's L2), then the
            // arrival count: the tile's last block reads every split's partial at device scope
            // (missing its own L2), adds them in split order from zero, as the separate reduction
            // does, and finishes the tile. Offsets are 32-bit (splits * M * N * 4 < 2^31, checked
            // by the host).
            const __amdgpu_buffer_rsrc_t prt = __builtin_amdgcn_make_buffer_rsrc(
                p.partial, (short)0, (int)(p.splits * p.M * p.N * 4), 0x00020000);
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int64_t row = m0 + wm * WTM + i * 16 + (lane & 15);
                    const int64_t col = n0 + wn * WTN + j * 16 + (lane >> 4) * 4;
                    if (row < p.M && col < p.N)
                        __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, acc[i][j]), prt,
                                                               (uint32_t)(((z * p.M + row) * p.N + col) * 4), 0,
                                                               CP_DEVICE_SCOPE);
                }
            __builtin_amdgcn_s_waitcnt(0x0f70);  // vmcnt(0): this wave's partials reached device scope
            __syncthreads();
            __shared__ int last;
            if (tid == 0) {
                const int old = __hip_atomic_fetch_add(arrive, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                last = old == p.splits - 1;
                if (last) __hip_atomic_store(arrive, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            }
            __syncthreads();
            if (!last) return;
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int j = 0; j < FN; ++j) {
                    const int64_t row = m0 + wm * WTM + i * 16 + (lane & 15);
                    const int64_t col = n0 + wn * WTN + j * 16 + (lane >> 4) * 4;
                    if (row >= p.M || col >= p.N) continue;
                    f32x4 sum = {0.f, 0.f, 0.f, 0.f};
                    for (int sp = 0; sp < p.splits; ++sp)
                        sum += sp == z ? acc[i][j]
                                       : __builtin_bit_cast(f32x4, __builtin_amdgcn_raw_buffer_load_b128(
                                                                       prt, (uint32_t)(((sp * p.M + row) * p.N + col) * 4),
                                                                       0, CP_DEVICE_SCOPE));
                    finish4<true, true>(p, sum, row, col, coff, 0);
                }
            return;
        }
    }
    if constexpr (XPOSE) {
        // The accumulator blocks hold C^T (B was the MFMA's row operand): lane l of block (i, j)
        // has output row i*16 + l%16 and its 4 consecutive columns j*16 + 4*(l/16) .. +3, so each
        // lane finishes one 4-column vector per block straight from its registers.
        if constexpr (KS) __syncthreads();  // row_inv
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) {
                const int rl = i * 16 + (lane & 15), cl = j * 16 + (lane >> 4) * 4;
                f32x4 v = acc[i][j];
                if constexpr (KS) v *= row_inv[wm * WTM + rl];
                finish4<true>(p, v, m0 + wm * WTM + rl, n0 + wn * WTN + cl, coff, z);
            }
    } else {
        // Epilogue through LDS: each wave stages half of its tile (WTM x WTN/2 f32) with static
        // register indices, then finishes it row-major with 4-column vectors (DUAL: the gate and
        // up waves of a row half finish their slice together).
        // Lane l of a 16x16 MFMA block holds rows 4*(l/16)+r (r = 0..3), column l%16.
        constexpr int EC = WTN / 2, EP = EC * 4 + 16;
        static_assert(4 * WTM * EP <= 2 * STAGE, "epilogue staging fits in the operand stages");
        __syncthreads();
        char *wl = smem + wave * (WTM * EP);
#pragma unroll
        for (int h = 0; h < 2; ++h) {
#pragma unroll
            for (int i = 0; i < FM; ++i)
#pragma unroll
                for (int jj = 0; jj < FN / 2; ++jj)
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const int rl = i * 16 + (lane >> 4) * 4 + r;
                        const int cl = jj * 16 + (lane & 15);
                        *(float *)(wl + rl * EP + cl * 4) = acc[i][h * (FN / 2) + jj][r];
                    }
            __syncthreads();
            if constexpr (DUAL) {
                const char *gl = smem + (wm * 2) * (WTM * EP), *ul = gl + WTM * EP;
                const int pt = wn * 64 + lane;
                for (int it = 0; it < (WTM * EC + 511) / 512; ++it) {
                    const int e = (it * 128 + pt) * 4;
                    if (WTM * EC % 512 != 0 && e >= WTM * EC) break;
                    const int rl = e / EC, cl = e % EC;
                    finish_swiglu4<true>(p, *(const f32x4 *)(gl + rl * EP + cl * 4),
                                         *(const f32x4 *)(ul + rl * EP + cl * 4), m0 + wm * WTM + rl,
                                         n0 + h * EC + cl, coff);
                }
            } else {
                for (int it = 0; it < WTM * EC / 256; ++it) {
                    const int e = (it * 64 + lane) * 4;
                    const int rl = e / EC, cl = e % EC;
                    f32x4 v = *(const f32x4 *)(wl + rl * EP + cl * 4);
                    if constexpr (KS) v *= row_inv[wm * WTM + rl];
                    finish4<true>(p, v, m0 + wm * WTM + rl, n0 + wn * WTN + h * EC + cl, coff, z);
                }
            }
            __syncthreads();
        }
    }
}

template <typename T, bool TA, bool TB, int BM, int BN, int WM, int WN, bool DUAL, int LM, bool KS = false, int PF = 1,
          bool XF = false>
__global__ __launch_bounds__(NTHREADS) void gemm_mfma(const GemmArgs p) {
    __shared__ __attribute__((aligned(16))) char smem[mfma_smem_bytes<T, TA, TB, BM, BN>()];
    gemm_mfma_block<T, TA, TB, BM, BN, WM, WN, DUAL, LM, KS, PF, XF>(p, blockIdx.x, blockIdx.y, smem);
}

typedef float f32x16 __attribute__((ext_vector_type(16)));

// Large-tile BF16 GEMM: 256x256 block tile, four waves each owning a 128x128 sub-tile built from
// 4x4 v_mfma_f32_32x32x16_bf16 blocks (256 FP32 accumulators per lane, held in AGPRs). Per 64-wide
// k-tile a wave issues 64 MFMAs against 32 128-bit LDS reads, half the LDS traffic per FLOP of the
// 64x64 wave tile of gemm_mfma.
//
// One wave per SIMD, so latency is hidden inside the wave by software pipelining:
//   * MFMA fragments are double-buffered: the LDS reads of k-step s+1 are in flight while the 16
//     MFMAs of step s issue;
//   * the global loads of tile t+1 are issued with the first MFMAs of tile t and written to the free
//     LDS stage during its last k-step;
//   * sched_group_barrier interleaves the DS reads, global loads and DS writes with the MFMAs.
// The loop body has no branches: the prefetch after the last tile re-reads the last tile (in
// bounds) and its LDS writes land in the stage nobody reads again.
template <bool TA, bool TB, bool EDGE, bool DUAL = false>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_256(const GemmArgs p) {
    using T = uint16_t;
    constexpr int BM = 256, BN = 256, BK = ET<T>::BK, WT = 128, F = 4;
    using OA = Operand<T, !TA, BM>;
    using OB = Operand<T, TB, BN>;
    // SwiGLU dual-B form: the B tile's rows 0..127 are 128 gate-weight rows and rows 128..255 the
    // same 128 rows of the up weight, so waves wn = 0 accumulate gate and wn = 1 up for one 256 x 128
    // output tile; the epilogue pairs them.
    using OBH = Operand<T, TB, BN / 2>;
    static_assert(!DUAL || (!TA && TB), "SwiGLU is Y = X.W^T");
    constexpr int SA = OA::STAGE_BYTES, SB = OB::STAGE_BYTES, STAGE = SA + SB;
    __shared__ __attribute__((aligned(16))) char smem[2 * STAGE];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    int tm, tn;
    map_tile(blockIdx.x, p.tiles_m, p.tiles_n, tm, tn);
    const int64_t z = blockIdx.y;
    const int64_t b = z % p.batch, split = z / p.batch;
    const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
    const T *A = (const T *)p.A + bo * p.sA_out + bi * p.sA_in;
    const T *B = (const T *)p.B + bo * p.sB_out + bi * p.sB_in;
    const int64_t coff = bo * p.sC_out + bi * p.sC_in;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (DUAL ? BN / 2 : BN);
    const T *B2 = DUAL ? (const T *)p.B2 + bo * p.sB_out + bi * p.sB_in : nullptr;

    if (p.causal != CAUSAL_NONE && n0 > m0 + BM - 1 + p.causal_offset) {
        if (p.causal == CAUSAL_WRITE) {
            for (int e = tid; e < BM * BN; e += NTHREADS) {
                const int64_t row = m0 + e / BN, col = n0 + e % BN;
                if (row < p.M && col < p.N) store_out(p.C, coff + row * p.ldc + col, -INFINITY, p.out_bf16);
            }
        }
        return;
    }

    int64_t kb = split * p.k_per_split;
    int64_t ke = min(p.K, kb + p.k_per_split);
    if (p.kmode == KMODE_LOWER) ke = min(ke, m0 + BM);
    if (p.kmode == KMODE_UPPER) kb = max(kb, (m0 / BK) * BK);
    const int ntiles = ke > kb ? (int)((ke - kb + BK - 1) / BK) : 0;

    const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    f32x16 acc[F][F];
#pragma unroll
    for (int i = 0; i < F; ++i)
#pragma unroll
        for (int j = 0; j < F; ++j) acc[i][j] = zero;

    if (ntiles > 0) {
        OA ga;
        std::conditional_t<DUAL, OBH, OB> gb;
        std::conditional_t<DUAL, OBH, char> gb2;
        u32x4 fa0[F], fb0[F], fa1[F], fb1[F];
        const int last = ntiles - 1;
        auto frags = [&](u32x4 (&fa)[F], u32x4 (&fb)[F], const char *st, int ks) {
#pragma unroll
            for (int i = 0; i < F; ++i) fa[i] = OA::frag32(st, wm * WT + i * 32, ks, lane);
#pragma unroll
            for (int j = 0; j < F; ++j) fb[j] = OB::frag32(st + SA, wn * WT + j * 32, ks, lane);
        };
        auto mfma16 = [&](const u32x4 (&fa)[F], const u32x4 (&fb)[F]) {
#pragma unroll
            for (int i = 0; i < F; ++i)
#pragma unroll
                for (int j = 0; j < F; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                        __builtin_bit_cast(bf16x8, fa[i]), __builtin_bit_cast(bf16x8, fb[j]), acc[i][j], 0, 0, 0);
        };
        // Tile k0: global loads into registers now, LDS writes in put().
        auto fetch = [&](int64_t k0) {
            constexpr int LM = EDGE ? LOAD_CHECKED : LOAD_EXACT;
            ga.template load<LM>(A, p.lda, m0, k0, p.M, ke, p.a_vec_ok, tid);
            gb.template load<LM>(B, p.ldb, n0, k0, p.N, ke, p.b_vec_ok, tid);
            if constexpr (DUAL) gb2.template load<LM>(B2, p.ldb, n0, k0, p.N, ke, p.b_vec_ok, tid);
        };
        auto put = [&](char *stage) {
            ga.store(stage, tid);
            gb.store(stage + SA, tid);
            if constexpr (DUAL) gb2.store(stage + SA + OBH::STAGE_BYTES, tid);
        };
        // DS writes per k-tile, spread over the 8 MFMA pairs of the last k-step (the dual halves
        // together issue what one 256-row B operand does).
        constexpr int DSW = (OA::ITERS * (OA::TRANSPOSE ? 8 : 1) + OB::ITERS * (OB::TRANSPOSE ? 8 : 1) + 7) / 8;
        constexpr int VMR = (OA::ITERS * OA::LOADS + OB::ITERS * OB::LOADS + 7) / 8;

        fetch(kb);
        put(smem);
        __syncthreads();
        frags(fa0, fb0, smem, 0);
        for (int t = 0; t < ntiles; ++t) {
            const char *cur = smem + (t & 1) * STAGE;
            char *nxt = smem + ((t + 1) & 1) * STAGE;
            // Tile t+1 (the last tile again at the end: in bounds, written to a dead stage).
            frags(fa1, fb1, cur, 1);
            fetch(kb + (int64_t)min(t + 1, last) * BK);
            mfma16(fa0, fb0);
            frags(fa0, fb0, cur, 2);
            mfma16(fa1, fb1);
            frags(fa1, fb1, cur, 3);
            mfma16(fa0, fb0);
            put(nxt);
            mfma16(fa1, fb1);
            if constexpr (!EDGE) {
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    __builtin_amdgcn_sched_group_barrier(sg::DS_READ, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(sg::VMEM_READ, VMR, 0);
                    __builtin_amdgcn_sched_group_barrier(sg::MFMA, 2, 0);
                }
#pragma unroll
                for (int g = 0; g < 16; ++g) {
                    __builtin_amdgcn_sched_group_barrier(sg::DS_READ, 1, 0);
                    __builtin_amdgcn_sched_group_barrier(sg::MFMA, 2, 0);
                }
#pragma unroll
                for (int g = 0; g < 8; ++g) {
                    __builtin_amdgcn_sched_group_barrier(sg::DS_WRITE, DSW, 0);
                    __builtin_amdgcn_sched_group_barrier(sg::MFMA, 2, 0);
                }
            }
            __syncthreads();
            frags(fa0, fb0, nxt, 0);
        }
    }
    __syncthreads();

    // Epilogue through LDS (free after the last barrier): each wave stages a quarter of its 128x128
    // tile (128 x 32 f32) with static register indices, then finishes it row-major with 4-column
    // vectors, so stores are coalesced and the accumulators never need dynamic indexing.
    // Lane l of a 32x32 block holds column l%32 and rows 8*(r/4) + 4*(l/32) + r%4, r = 0..15.
    constexpr int EC = 32, EP = EC * 4 + 16;
    static_assert(4 * WT * EP <= 2 * STAGE, "epilogue staging fits in the operand stages");
    char *wl = smem + wave * (WT * EP);
#pragma unroll
    for (int h = 0; h < F; ++h) {
#pragma unroll
        for (int i = 0; i < F; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r) {
                const int rl = i * 32 + (r >> 2) * 8 + (lane >> 5) * 4 + (r & 3);
                const int cl = lane & 31;
                *(float *)(wl + rl * EP + cl * 4) = acc[i][h][r];
            }
        __syncthreads();
        if constexpr (DUAL) {
            // The two waves of row half wm (gate: wn = 0, up: wn = 1) finish its 128 x 32 slice.
            const char *gl = smem + (wm * 2) * (WT * EP), *ul = gl + WT * EP;
            const int pt = wn * 64 + lane;
            for (int it = 0; it < WT * EC / 512; ++it) {
                const int e = (it * 128 + pt) * 4;
                const int rl = e / EC, cl = e % EC;
                finish_swiglu4<EDGE>(p, *(const f32x4 *)(gl + rl * EP + cl * 4), *(const f32x4 *)(ul + rl * EP + cl * 4),
                                     m0 + wm * WT + rl, n0 + h * EC + cl, coff);
            }
        } else {
            for (int it = 0; it < WT * EC / 256; ++it) {
                const int e = (it * 64 + lane) * 4;
                const int rl = e / EC, cl = e % EC;
                const f32x4 v = *(const f32x4 *)(wl + rl * EP + cl * 4);
                finish4<EDGE>(p, v, m0 + wm * WT + rl, n0 + wn * WT + h * EC + cl, coff, z);
            }
        }
        __syncthreads();
    }
}

// BF16 256x256x64 GEMM with direct global -> LDS loads (buffer_load_dwordx4 ... lds): the wave never
// holds operand tiles in registers and issues no LDS writes of its own, so a k-tile costs it 16
// load instructions (their offsets fixed for the whole k loop, the k position in the scalar offset)
// besides its fragment reads and 64 MFMAs (v_mfma_f32_32x32x16_bf16, 128x128 per wave). Two stages
// in two LDS objects (so the compiler can see that loads into one never alias reads of the other);
// the loads of tile t+2 are issued right after the barrier that ends the reads of tile t's stage,
// so they have a whole k-tile to land before the wait that precedes the next barrier.
//
// Each operand's stage (32 KB) is laid out by its global layout:
//   k-contiguous (A not transposed, B transposed): [256 rows][64 k], 128-byte rows, the 16-byte
//     chunk c of row r at position c ^ ((r >> 1) & 7); a load instruction fills 8 rows (lane L:
//     row L / 8, position L % 8); a fragment (32 rows x 8 k) is one ds_read_b128 per lane, the 16
//     lanes served together hitting 16 distinct 16-byte bank groups.
//   mn-contiguous (A transposed, B not): [64 k][256 rows], 512-byte k-rows, chunk c of k-row q at
//     position c ^ (4 (q & 3)); a load instruction fills 2 k-rows (lane L: k-row L / 32, position
//     L % 32); a fragment is two ds_read_tr16_b64 per lane, each giving a 16-lane group a 16 x 4
//     (rows x k) block transposed: lane j of the group points at the 4 rows 4 (j % 4) .. +3 of
//     k-row j / 4 and receives 4 consecutive k of row j. The 32 lanes served together hit 16
//     distinct 16-byte bank groups.
// The 256 x 128 form (FB = 2: each wave 128 x 64) stages 128 B rows: 4 load instructions per wave,
// an mn-contiguous k-row of 256 bytes (16 chunks, the same XOR, 4 k-rows per load instruction).
// Whole tiles only (M a multiple of 256, N of the tile width, K of 128); no k limits or masked
// epilogues.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t dtl_rsrc(const void *base, int64_t bytes) {
    const int n = bytes > 0x7fffffff ? 0x7fffffff : (int)bytes;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void *>(base), (short)0, n, 0x00020000);
}

typedef __attribute__((address_space(3))) void lds_void_t;
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) s16x4 lds_s16x4_t;

// p through an empty asm: the compiler no longer knows which LDS object it points into.
__device__ __forceinline__ lds_void_t *opaque_lds(lds_void_t *p) {
    uint32_t x = (uint32_t)(uintptr_t)p;
    asm("" : "+s"(x));
    return (lds_void_t *)(uintptr_t)x;
}

template <bool KCONTIG, int ROWS = 256>
struct DtlOperand {
    static constexpr int BK = 64;
    // Load instructions per wave per k-tile (each fills 1 KB: 8 k-contiguous rows, or 1024 / (2
    // ROWS) k-rows of an mn-contiguous operand).
    static constexpr int NI = ROWS / 32;
    static constexpr int RB = ROWS * 2;     // bytes per k-row (mn-contiguous)
    static constexpr int CPR = ROWS / 8;    // 16-byte chunks per k-row
    static_assert(ROWS == 256 || ROWS == 128, "256 or 128 rows");
    __amdgpu_buffer_rsrc_t rsrc;
    uint32_t voff[NI];
    uint32_t kstride;  // bytes per k of the global operand (2 for k-contiguous, 2 ld otherwise)

    // base: element (row 0, k kb) of this block; krange: k extent of this block's split. A
    // k-contiguous operand may take the rows from `row_shift` on from a second matrix (the up
    // weight of the SwiGLU dual form: this wave's rows are then rows r - row_shift of `base`).
    __device__ __forceinline__ void init(const uint16_t *base, int64_t ld, int64_t krange, int wave, int lane,
                                         int row_shift = 0) {
        if constexpr (KCONTIG) {
            rsrc = dtl_rsrc(base, (int64_t)(ROWS - row_shift) * ld * 2);
            kstride = 2;
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const int r = 8 * (NI * wave + j) + (lane >> 3);
                const int c = (lane & 7) ^ ((r >> 1) & 7);
                voff[j] = (uint32_t)(((r - row_shift) * ld + c * 8) * 2);
            }
        } else {
            rsrc = dtl_rsrc(base, krange * ld * 2);
            kstride = (uint32_t)(ld * 2);
#pragma unroll
            for (int j = 0; j < NI; ++j) {
                const int q = (64 / CPR) * (NI * wave + j) + lane / CPR;
                const int c = (lane % CPR) ^ (4 * (q & 3));
                voff[j] = (uint32_t)((q * ld + c * 8) * 2);
            }
        }
    }

    // The k-tile starting kk elements into the split, into `stage`. opaque (a constant at each
    // call): the LDS address reaches the load through an empty asm, so the compiler cannot tie
    // the load to an LDS object and inserts no waits of its own before LDS reads (which, not
    // knowing which stage a pending load writes, would wait for all of them); the caller's
    // explicit waits then order them.
    __device__ __forceinline__ void issue(char *stage, int64_t kk, int wave, bool opaque) const {
        const uint32_t soff = (uint32_t)(kk * kstride);
#pragma unroll
        for (int j = 0; j < NI; ++j) {
            lds_void_t *dst = (lds_void_t *)(stage + (NI * wave + j) * 1024);
            if (opaque) dst = opaque_lds(dst);
            __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, dst, 16, voff[j], soff, 0, 0);
        }
    }

    // Fragment (rows row .. row + 31, k 16 ks .. +15) of a 32x32x16 MFMA operand: lane l holds row
    // row + l % 32 at k 16 ks + 8 (l / 32) .. +7.
    __device__ __forceinline__ static u32x4 frag(const char *st, int row, int ks, int lane) {
        if constexpr (KCONTIG) {
            const int fr = lane & 31;
            const int y = (lane >> 5) ^ ((fr >> 1) & 7);
            return *(const u32x4 *)(st + (row + fr) * 128 + (((2 * ks) ^ y) * 16));
        } else {
            const int g = lane >> 4, j = lane & 15;
            const int n = row + 16 * (g & 1);           // first row of this group's 16
            const int q = 16 * ks + 8 * (g >> 1) + (j >> 2);  // k-row of this lane's chunk
            const int cbyte = n * 2 + 8 * (j & 3);       // byte of the chunk within the k-row
            const int off = (((cbyte >> 4) ^ (4 * (q & 3))) << 4) + (cbyte & 15);
            const s16x4 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(st + q * RB + off));
            const s16x4 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_t *)(st + (q + 4) * RB + off));
            u32x4 v;
            v[0] = (uint32_t)(uint16_t)lo[0] | ((uint32_t)(uint16_t)lo[1] << 16);
            v[1] = (uint32_t)(uint16_t)lo[2] | ((uint32_t)(uint16_t)lo[3] << 16);
            v[2] = (uint32_t)(uint16_t)hi[0] | ((uint32_t)(uint16_t)hi[1] << 16);
            v[3] = (uint32_t)(uint16_t)hi[2] | ((uint32_t)(uint16_t)hi[3] << 16);
            return v;
        }
    }
};

// The k loop of one tile: acc = op(A)[m0.., kb..] . op(B)[.., n0..] over `ntiles` k-tiles (even).
// A and B point at element (row 0, k kb) of the tile's operands; `krange` bounds an mn-contiguous
// operand's buffer. The caller synchronises the block before (the stages may still be read) and
// after (the epilogue reuses them).
// s_waitcnt immediate: vmcnt(vm) lgkmcnt(lgkm), expcnt not waited on.
constexpr int waitcnt_imm(int vm, int lgkm) { return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | (lgkm << 8); }

template <bool TA, bool TB, bool DUAL, int FB, bool OPAQUE = (FB == 2), int FA = 4, int NSX = 0>
__device__ __forceinline__ void dtl_tile(const GemmArgs &p, char *__restrict__ st0, char *__restrict__ st1,
                                         char *__restrict__ st2, char *__restrict__ st3, const uint16_t *A,
                                         const uint16_t *B, int64_t krange, int ntiles, f32x16 (&acc)[FA][FB],
                                         int wave, int lane) {
    // OPAQUE: the direct loads' LDS addresses hidden from the compiler (needed whenever the
    // stages share one LDS object or are three or more: then only the explicit waits order the
    // loads). FA / FB: 32-row A / 32-column B fragments per wave. FA = 4, FB = 4: 256 x 256 tile,
    // 128 x 128 per wave, two 64 KB stages; FA = 4, FB = 2: 256 x 128 tile, 128 x 64 per wave,
    // three 48 KB stages, so that loads run two k-tiles ahead of a k-tile that takes half as long;
    // FA = 2, FB = 2: 128 x 128 tile, 64 x 64 per wave, NSX stages of 32 KB (a k-tile is a quarter
    // of the 256 x 256 one: more stages keep the same load latency covered).
    constexpr int BN = FB * 64, BK = 64, WT = FA * 32, F = FA;
    constexpr int NS = NSX ? NSX : FB == 2 ? 3 : 2;
    static_assert(NS >= 2 && NS <= 4 && (NS == 2 || OPAQUE), "two to four stages; three or more need OPAQUE");
    constexpr int TILE = FA * 64 * BK * 2;
    using OA = DtlOperand<!TA, FA * 64>;
    using OB = DtlOperand<TB, BN>;
    const int wm = wave >> 1, wn = wave & 1;
    const f32x16 zero = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < F; ++i)
#pragma unroll
        for (int j = 0; j < FB; ++j) acc[i][j] = zero;
    if (ntiles <= 0) return;
    OA oa;
    OB ob;
    oa.init(A, p.lda, krange, wave, lane);
    ob.init(B, p.ldb, krange, wave, lane, DUAL && wave >= 2 ? BN / 2 : 0);
    const int last = ntiles - 1;
    auto issue = [&](int t, char *stage) {
        const int64_t kk = (int64_t)min(t, last) * BK;
        oa.issue(stage, kk, wave, OPAQUE);
        ob.issue(stage + TILE, kk, wave, OPAQUE);
    };
    u32x4 fa0[F], fb0[FB], fa1[F], fb1[FB];
    auto frags = [&](u32x4 (&fa)[F], u32x4 (&fb)[FB], const char *st, int ks) {
#pragma unroll
        for (int i = 0; i < F; ++i) fa[i] = OA::frag(st, wm * WT + i * 32, ks, lane);
#pragma unroll
        for (int j = 0; j < FB; ++j) fb[j] = OB::frag(st + TILE, wn * (FB * 32) + j * 32, ks, lane);
    };
    auto mfma16 = [&](const u32x4 (&fa)[F], const u32x4 (&fb)[FB]) {
#pragma unroll
        for (int i = 0; i < F; ++i)
#pragma unroll
            for (int j = 0; j < FB; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(
                    __builtin_bit_cast(bf16x8, fa[i]), __builtin_bit_cast(bf16x8, fb[j]), acc[i][j], 0, 0, 0);
    };
    // DS reads per MFMA pair (a k-step's fragment set is F + FB fragments, an mn-contiguous one
    // two reads each; the k-step has F FB / 2 MFMA pairs), and load instructions per pair in the
    // k-step that issues them.
    constexpr int PAIRS = F * FB / 2;
    constexpr int DSR = (F * (TA ? 2 : 1) + FB * (TB ? 1 : 2) + PAIRS - 1) / PAIRS;
    constexpr int VMR = (OA::NI + OB::NI + PAIRS - 1) / PAIRS;
    // Load instructions a wave issues per k-tile: with three stages the wait before the barrier
    // lets the newest k-tile's loads stay in flight.
    constexpr int NLOAD = OA::NI + OB::NI;
    constexpr int WAIT_NEXT = waitcnt_imm((NS - 2) * NLOAD, 0);
    // Tile t from `cur` (its k-step 0 fragments already in fa0/fb0); tile t+1 has been streaming
    // into `nxt` (and, with three stages, tile t+2 into the third); the loads of tile t+NS go into
    // `cur` once every wave has passed the barrier.
    auto body = [&](char *cur, const char *nxt, int t) {
        frags(fa1, fb1, cur, 1);
        mfma16(fa0, fb0);
        frags(fa0, fb0, cur, 2);
        mfma16(fa1, fb1);
        frags(fa1, fb1, cur, 3);
        mfma16(fa0, fb0);
        // k-steps 0..2, each step's MFMAs interleaved with the next step's fragment reads.
#pragma unroll
        for (int g = 0; g < 3 * PAIRS; ++g) {
            __builtin_amdgcn_sched_group_barrier(sg::DS_READ, DSR, 0);
            __builtin_amdgcn_sched_group_barrier(sg::MFMA, 2, 0);
        }
        __builtin_amdgcn_s_waitcnt(WAIT_NEXT);  // lgkmcnt(0): `cur` read; tile t+1 landed
        if constexpr (NS == 2) {
            __syncthreads();
        } else {
            // No release fence: at workgroup scope it would also wait for the newest tile's
            // loads (vmcnt(0)). The explicit wait above has completed this wave's reads of `cur`,
            // and the barrier keeps them ahead of the loads into it; the acquire fence keeps the
            // reads of `nxt` behind the barrier.
            __builtin_amdgcn_s_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
        }
        issue(t + NS, cur);
        // k-step 3 with the next tile's first fragment reads and the loads of tile t+NS.
        frags(fa0, fb0, nxt, 0);
        mfma16(fa1, fb1);
#pragma unroll
        for (int g = 0; g < PAIRS; ++g) {
            __builtin_amdgcn_sched_group_barrier(sg::DS_READ, DSR, 0);
            __builtin_amdgcn_sched_group_barrier(sg::VMEM_READ, VMR, 0);
            __builtin_amdgcn_sched_group_barrier(sg::MFMA, 2, 0);
        }
    };
    if constexpr (NS == 2) {
        issue(0, st0);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));
        __syncthreads();
        issue(1, st1);
        frags(fa0, fb0, st0, 0);
        // An even number of k-tiles (dtl_applicable): no odd tail body, whose prefetched fragments
        // would stay live past the loop and spill.
        for (int t = 0; t < ntiles; t += 2) {
            body(st0, st1, t);
            body(st1, st0, t + 1);
        }
    } else if constexpr (NS == 3) {
        issue(0, st0);
        issue(1, st1);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(NLOAD, 15));  // tile 0 landed
        __syncthreads();
        issue(2, st2);
        frags(fa0, fb0, st0, 0);
        // Any number of k-tiles (the 256 x 128 tile has registers to spare for the tail).
        for (int t = 0;; t += 3) {
            body(st0, st1, t);
            if (t + 1 >= ntiles) break;
            body(st1, st2, t + 1);
            if (t + 2 >= ntiles) break;
            body(st2, st0, t + 2);
            if (t + 3 >= ntiles) break;
        }
    } else {
        issue(0, st0);
        issue(1, st1);
        issue(2, st2);
        __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * NLOAD, 15));  // tile 0 landed
        __syncthreads();
        issue(3, st3);
        frags(fa0, fb0, st0, 0);
        for (int t = 0;; t += 4) {
            body(st0, st1, t);
            if (t + 1 >= ntiles) break;
            body(st1, st2, t + 1);
            if (t + 2 >= ntiles) break;
            body(st2, st3, t + 2);
            if (t + 3 >= ntiles) break;
            body(st3, st0, t + 3);
            if (t + 4 >= ntiles) break;
        }
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 15));  // the loads into dead stages have landed
}

// Epilogue of one tile of gemm_bf16_dtl (begins with a block barrier: the stages are reused).
// Passes of 128 x 64 columns per wave (two with FB = 4, one with FB = 2), each wave staging 32 KB
// as two 16 KB halves of 64 rows: FB = 4, waves 0-1 in st0 and 2-3 in st1 (64 KB stages); FB = 2,
// waves 0-2 in st0, st1, st2 and wave 3 in the 16 KB tails of st0 and st1 (48 KB stages). 16 lanes
// then read a whole 256-byte staged row, so every store covers whole 128-byte lines of a BF16 (or
// FP32) output row. Row r's columns sit at c ^ 32 ((r >> 2) & 1): the two rows one accumulator
// write instruction touches (4 apart) then fall in different banks. In the SwiGLU form the gate
// wave (wn = 0) and the up wave (wn = 1) of a row half stage the same output columns and then
// finish 64 rows each of the pair.
template <bool DUAL, int FB, int FA = 4>
__device__ __forceinline__ void dtl_epilogue(const GemmArgs &p, char *st0, char *st1, char *st2,
                                             const f32x16 (&acc)[FA][FB], int64_t m0, int64_t n0, int64_t coff,
                                             int64_t z, int wave, int lane) {
    static_assert(!DUAL || (FB == 4 && FA == 4), "the SwiGLU form pairs 128-column gate and up waves");
    constexpr int WT = FA * 32, F = FA, NH = FA / 2;  // NH: 64-row halves per wave
    constexpr int STAGE = FA == 2 ? 2 * 128 * 64 * 2 : FB == 4 ? 2 * 256 * 64 * 2 : (256 + 128) * 64 * 2;
    constexpr int EC2 = 64, EP2 = EC2 * 4, HALF = 64 * EP2;
    static_assert(FA == 2 ? 2 * HALF <= STAGE : FB == 4 ? 4 * HALF <= STAGE : 3 * HALF <= STAGE,
                  "epilogue staging fits in the stages");
    const int wm = wave >> 1, wn = wave & 1;
    __syncthreads();
    char *lo, *hi;  // this wave's staging for rows 0-63 and 64-127 of its 128 (FA = 2: 64 rows, lo)
    if constexpr (FA == 2) {
        // two 16 KB halves in each of st0 (waves 0-1) and st1 (waves 2-3)
        lo = (wave < 2 ? st0 : st1) + (wave & 1) * HALF;
        hi = lo;
    } else if constexpr (FB == 4) {
        lo = (wave < 2 ? st0 : st1) + (wave & 1) * (2 * HALF);
        hi = lo + HALF;
    } else {
        (void)st2;
        lo = wave == 0 ? st0 : wave == 1 ? st1 : wave == 2 ? st2 : st0 + 2 * HALF;
        hi = wave == 3 ? st1 + 2 * HALF : lo + HALF;
    }
    // A lane's accumulator rows all have bit 2 equal to lane / 32, so its swizzle is per lane.
    const int lane_off = (lane >> 5) * 4 * EP2 + (lane & 31) * 4 + ((lane >> 5) << 7);
#pragma unroll
    for (int hp = 0; hp < FB / 2; ++hp) {
#pragma unroll
        for (int hh = 0; hh < 2; ++hh)
#pragma unroll
            for (int i = 0; i < F; ++i)
#pragma unroll
                for (int r = 0; r < 16; ++r) {
                    // row less the lane's 4 (lane / 32), within the half (i < 2: rows 0-63)
                    const int rr = (i & 1) * 32 + (r >> 2) * 8 + (r & 3);
                    // column hh * 32 + lane % 32, bit 5 flipped for odd lane / 32: one XOR per lane,
                    // folded into lane_off for hh = 0 and undone (^ 32 = +-32) for hh = 1.
                    float *dst = (float *)((i < 2 ? lo : hi) + lane_off) + rr * (EP2 / 4) +
                                 (hh ? (((lane >> 5) & 1) ? -32 : 32) : 0);
                    *dst = acc[i][2 * hp + hh][r];
                }
        __syncthreads();
        // Lane reads row 4 it + lane / 16 of a half, columns cl .. cl + 3; bit 2 of the row is it & 1.
        const int cl = (lane & 15) * 4;
        if constexpr (DUAL) {
            // The gate wave's staging (wn = 0) and the up wave's (wn = 1) of this row half are
            // consecutive 32 KB in one stage.
            const char *gl = wm == 0 ? st0 : st1, *ul = gl + 2 * HALF;
            const int64_t col = n0 + hp * EC2 + cl;
            if (p.c_vec_ok && p.out_bf16) {
                // BF16 outputs (as finish_swiglu4's vector path): the bias and the row pointers
                // once per pass, then per row h = silu(g) u with g, u = alpha acc + bias.
                f32x4 bg = {0.f, 0.f, 0.f, 0.f}, bu = {0.f, 0.f, 0.f, 0.f};
                if (p.has_bias) {
                    bg = f32x4{p.bias[col], p.bias[col + 1], p.bias[col + 2], p.bias[col + 3]};
                    bu = f32x4{p.bias[p.N + col], p.bias[p.N + col + 1], p.bias[p.N + col + 2], p.bias[p.N + col + 3]};
                }
                const int64_t idx = coff + (m0 + wm * WT + 4 * (wn * 16) + (lane >> 4)) * p.ldc + col;
                uint16_t *hd = (uint16_t *)p.C + idx;
                uint16_t *gd = p.G ? (uint16_t *)p.G + idx : nullptr;
                uint16_t *ud = p.U ? (uint16_t *)p.U + idx : nullptr;
                const int64_t step = 4 * p.ldc;
#pragma unroll 4
                for (int it = wn * 16; it < wn * 16 + 16; ++it) {
                    const int off = (4 * it + (lane >> 4)) * EP2 + ((cl ^ ((it & 1) << 5)) * 4);
                    const f32x4 g = *(const f32x4 *)(gl + off) * p.alpha + bg;
                    const f32x4 u = *(const f32x4 *)(ul + off) * p.alpha + bu;
                    f32x4 h;
#pragma unroll
                    for (int e = 0; e < 4; ++e) h[e] = silu(g[e]) * u[e];
                    *(u32x2 *)hd = u32x2{pack_bf16x2(h[0], h[1]), pack_bf16x2(h[2], h[3])};
                    if (gd) *(u32x2 *)gd = u32x2{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3])};
                    if (ud) *(u32x2 *)ud = u32x2{pack_bf16x2(u[0], u[1]), pack_bf16x2(u[2], u[3])};
                    hd += step;
                    if (gd) gd += step;
                    if (ud) ud += step;
                }
            } else {
#pragma unroll 4
                for (int it = wn * 16; it < wn * 16 + 16; ++it) {
                    const int rl = 4 * it + (lane >> 4);
                    const int off = rl * EP2 + ((cl ^ ((it & 1) << 5)) * 4);
                    finish_swiglu4<false>(p, *(const f32x4 *)(gl + off), *(const f32x4 *)(ul + off),
                                          m0 + wm * WT + rl, col, coff);
                }
            }
        } else {
            const int64_t col = n0 + wn * (FB * 32) + hp * EC2 + cl;
            auto staged = [&](int h, int it) {
                return *(const f32x4 *)((h ? hi : lo) + (4 * it + (lane >> 4)) * EP2 + ((cl ^ ((it & 1) << 5)) * 4));
            };
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const int64_t row0 = m0 + wm * WT + h * 64 + (lane >> 4);
                if (p.splits > 1) {
                    // split-K partial sums: plain f32 rows of N
                    float *dst = p.partial + (z * p.M + row0) * p.N + col;
#pragma unroll 4
                    for (int it = 0; it < 16; ++it, dst += 4 * p.N) *(f32x4 *)dst = staged(h, it);
                } else if (p.c_vec_ok && !p.row_scale && p.beta == 0.f && !p.rope_table) {
                    // the common epilogue: alpha (and a column bias) only, with one base pointer per half
                    f32x4 bias = {0.f, 0.f, 0.f, 0.f};
                    if (p.has_bias) bias = f32x4{p.bias[col], p.bias[col + 1], p.bias[col + 2], p.bias[col + 3]};
                    const int64_t idx = coff + row0 * p.ldc + col;
                    if (p.out_bf16) {
                        uint16_t *dst = (uint16_t *)p.C + idx;
#pragma unroll 4
                        for (int it = 0; it < 16; ++it, dst += 4 * p.ldc) {
                            const f32x4 v = staged(h, it) * p.alpha + bias;
                            *(u32x2 *)dst = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
                        }
                    } else {
                        float *dst = (float *)p.C + idx;
#pragma unroll 4
                        for (int it = 0; it < 16; ++it, dst += 4 * p.ldc) *(f32x4 *)dst = staged(h, it) * p.alpha + bias;
                    }
                } else {
#pragma unroll 4
                    for (int it = 0; it < 16; ++it)
                        finish4<false>(p, staged(h, it), row0 + 4 * it, col, coff, z);
                }
            }
        }
        __syncthreads();
    }
}

// One block of gemm_bf16_dtl: output tile `tile` (in map_tile order) of batch-and-split index z.
// DUAL (SwiGLU, Y = X.W^T only): the B stage's rows 0..127 are 128 gate-weight rows (loaded by
// waves 0-1) and rows 128..255 the same rows of the up weight (waves 2-3), so waves wn = 0
// accumulate gate and wn = 1 up for one 256 x 128 output tile; the epilogue pairs them. FB = 2:
// a 256 x 128 output tile (twice the tiles where 256 x 256 would leave CUs idle), with three
// stages of 48 KB.
template <bool TA, bool TB, bool DUAL, int FB, bool OPAQUE = (FB == 2), int FA = 4, int NS = 0>
__device__ __forceinline__ void dtl_block(const GemmArgs &p, int tile, int64_t z, char *st0, char *st1, char *st2,
                                          char *st3 = nullptr) {
    static_assert(!DUAL || (!TA && TB), "SwiGLU is Y = X.W^T");
    using T = uint16_t;
    constexpr int BM = FA * 64, BN = FB * 64, BK = 64, F = FA;
    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int tm, tn;
    map_tile(tile, p.tiles_m, p.tiles_n, tm, tn);
    const int64_t b = z % p.batch, split = z / p.batch;
    const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
    const int64_t m0 = (int64_t)tm * BM, n0 = (int64_t)tn * (DUAL ? BN / 2 : BN);
    const int64_t kb = split * p.k_per_split;
    const int64_t ke = min(p.K, kb + p.k_per_split);
    const T *A = (const T *)p.A + bo * p.sA_out + bi * p.sA_in + (TA ? kb * p.lda + m0 : m0 * p.lda + kb);
    const T *Bm = (const T *)(DUAL && wave >= 2 ? p.B2 : p.B);
    const T *B = Bm + bo * p.sB_out + bi * p.sB_in + (TB ? n0 * p.ldb + kb : kb * p.ldb + n0);
    f32x16 acc[F][FB];
    dtl_tile<TA, TB, DUAL, FB, OPAQUE, FA, NS>(p, st0, st1, st2, st3, A, B, ke - kb,
                                               ke > kb ? (int)((ke - kb) / BK) : 0, acc, wave, lane);
    dtl_epilogue<DUAL, FB, FA>(p, st0, st1, st2, acc, m0, n0, bo * p.sC_out + bi * p.sC_in, z, wave, lane);
}

template <bool TA, bool TB, bool DUAL = false, int FB = 4>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_dtl(const GemmArgs p) {
    constexpr int STAGE = (256 + (FB == 4 ? 256 : 128)) * 64 * 2;
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[FB == 2 ? STAGE : 16];  // FB = 2 only
    dtl_block<TA, TB, DUAL, FB>(p, blockIdx.x, blockIdx.y, st0, st1, st2);
}

// 128 x 128 tiles (64 x 64 per wave), four stages of 32 KB: for shapes whose 256-wide tiles would
// leave CUs idle (2048^3: 256 tiles, one per CU, where 256 x 256 gives 64). Each stage is an LDS
// object of its own: with the four in one object the compiler put a wait for every outstanding
// direct load (vmcnt(0)) before each transposing fragment read (ds_read_b64_tr_b16), so the loads
// of an mn-contiguous operand never ran ahead of the k-tile being multiplied.
constexpr int DTL128_STAGES = 4;
template <bool TA, bool TB>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_dtl128(const GemmArgs p) {
    constexpr int STAGE = 2 * 128 * 64 * 2;
    static_assert(DTL128_STAGES == 4, "four stage objects");
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    __shared__ __attribute__((aligned(1024))) char st2[STAGE];
    __shared__ __attribute__((aligned(1024))) char st3[STAGE];
    dtl_block<TA, TB, false, 2, true, 2, DTL128_STAGES>(p, blockIdx.x, blockIdx.y, st0, st1, st2, st3);
}

// Several independent GEMMs of one layout in one launch. Workgroup w runs on XCD w % 8, and each
// XCD has its own L2, so the blocks are scheduled per XCD: XCD x runs blocks j = 0 .. xn[x] - 1
// (workgroup j * 8 + x), an equal share of the group's tiles x splits, as contiguous chunks. Chunk c
// gives blocks jstart.. of its XCD the tiles t0, t0 + 1, ... (grouped raster order) of split `split`
// of problem gi, until the next chunk of that XCD starts. A problem's split then sits on one XCD
// (or two, where a share ends inside it), and its operand panels are fetched into one L2 instead of
// eight.
constexpr int GEMM_GROUP_MAX = 8;
constexpr int GROUP_CHUNKS = 96;
struct GroupChunk {
    uint16_t jstart;
    uint8_t gi, split;
    uint16_t t0, unused;
};
struct GemmGroupArgs {
    GemmArgs g[GEMM_GROUP_MAX];
    int *arrive;                         // FP32 groups: the split-K arrival counters (zero),
    int cstart[GEMM_GROUP_MAX + 1];      // problem g's tiles at arrive[cstart[g]] ..
    int count;
    uint16_t xn[8];                      // blocks of XCD x
    uint16_t xstart[9];                  // its chunks: chunk[xstart[x]] .. chunk[xstart[x + 1] - 1]
    GroupChunk chunk[GROUP_CHUNKS];
};

// The map_tile index whose tile is number r of the grouped raster order (map_tile's XCD remap
// undone: the group's schedule has already placed the block on its XCD).
__device__ __forceinline__ int raster_pid(int r, int total) {
    if (total % 8 != 0) return r;
    const int q = total / 8;
    return (r % q) * 8 + r / q;
}

// This block's problem, split and map_tile index under the group's XCD schedule; false for a block
// past its XCD's share.
__device__ __forceinline__ bool group_block(const GemmGroupArgs &grp, int &gi, int &split, int &tile) {
    const int x = (int)blockIdx.x & 7, j = (int)blockIdx.x >> 3;
    if (j >= grp.xn[x]) return false;
    int c = grp.xstart[x];
    while (c + 1 < grp.xstart[x + 1] && grp.chunk[c + 1].jstart <= j) ++c;
    gi = grp.chunk[c].gi;
    split = grp.chunk[c].split;
    const GemmArgs &p = grp.g[gi];
    tile = raster_pid(grp.chunk[c].t0 + (j - grp.chunk[c].jstart), p.tiles_m * p.tiles_n);
    return true;
}

// BF16: 256 x 256 direct-to-LDS tiles, batch 1, no split-K, one round of CUs.
template <bool TA, bool TB>
__global__ __launch_bounds__(NTHREADS) __attribute__((amdgpu_waves_per_eu(1, 1)))
void gemm_bf16_dtl_group(const GemmGroupArgs grp) {
    constexpr int STAGE = 512 * 64 * 2;
    __shared__ __attribute__((aligned(1024))) char st0[STAGE];
    __shared__ __attribute__((aligned(1024))) char st1[STAGE];
    int gi, split, tile;
    if (!group_block(grp, gi, split, tile)) return;
    dtl_block<TA, TB, false, 4>(grp.g[gi], tile, 0, st0, st1, st0);
}

// FP32: 64 x 64 tiles, batch 1, one split count for the group. Split-K partial sums go to each
// problem's own region, and each tile's last block to arrive adds its splits and finishes it.
template <bool TA, bool TB, int LM>
__global__ __launch_bounds__(NTHREADS) void gemm_f32_group(const GemmGroupArgs grp) {
    __shared__ __attribute__((aligned(16))) char smem[mfma_smem_bytes<float, TA, TB, 64, 64>()];
    int gi, split, tile;
    if (!group_block(grp, gi, split, tile)) return;
    gemm_mfma_block<float, TA, TB, 64, 64, 2, 2, false, LM, false, 2, false, true>(grp.g[gi], tile, split, smem,
                                                                                grp.arrive + grp.cstart[gi] + tile);
}

// Deterministic split-K reduction: partial sums are added in split order.
__global__ __launch_bounds__(256) void splitk_reduce(const GemmArgs p) {
    const int64_t total = p.batch * p.M * p.N;
    const int64_t mn = p.M * p.N;
    for (int64_t e = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e < total;
         e += (int64_t)gridDim.x * blockDim.x) {
        const int64_t b = e / mn, rem = e % mn, row = rem / p.N, col = rem % p.N;
        float s = 0.f;
        for (int sp = 0; sp < p.splits; ++sp) s += p.partial[(int64_t)sp * total + e];
        const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
        finish_store(p, p.C, bo * p.sC_out + bi * p.sC_in + row * p.ldc + col, s, row, col);
    }
}

// The same reduction 4 columns per thread (N % 4 == 0): 16-byte partial loads and the vector
// epilogue. Splits are summed in the same order, so results equal the scalar form's.
__global__ __launch_bounds__(256) void splitk_reduce4(const GemmArgs p) {
    const int64_t total = p.batch * p.M * p.N;
    const int64_t mn = p.M * p.N, total4 = total / 4;
    for (int64_t e4 = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; e4 < total4;
         e4 += (int64_t)gridDim.x * blockDim.x) {
        const int64_t e = e4 * 4;
        const int64_t b = e / mn, rem = e % mn, row = rem / p.N, col = rem % p.N;
        f32x4 s = {0.f, 0.f, 0.f, 0.f};
        for (int sp = 0; sp < p.splits; ++sp) s += *(const f32x4 *)(p.partial + (int64_t)sp * total + e);
        const int64_t bo = b / p.batch_inner, bi = b % p.batch_inner;
        finish4<false, true>(p, s, row, col, bo * p.sC_out + bi * p.sC_in, 0);
    }
}

struct TileCfg {
    int bm, bn;
};

template <bool EDGE>
void launch_bf16_256_e(bool ta, bool tb, const GemmArgs &a, dim3 grid, hipStream_t s) {
    if (a.dual) hipLaunchKernelGGL((gemm_bf16_256<false, true, EDGE, true>), grid, dim3(NTHREADS), 0, s, a);
    else if (!ta && !tb) hipLaunchKernelGGL((gemm_bf16_256<false, false, EDGE>), grid, dim3(NTHREADS), 0, s, a);
    else if (!ta && tb) hipLaunchKernelGGL((gemm_bf16_256<false, true, EDGE>), grid, dim3(NTHREADS), 0, s, a);
    else if (ta && !tb) hipLaunchKernelGGL((gemm_bf16_256<true, false, EDGE>), grid, dim3(NTHREADS), 0, s, a);
    else hipLaunchKernelGGL((gemm_bf16_256<true, true, EDGE>), grid, dim3(NTHREADS), 0, s, a);
}

// Tiles need no bounds checks when every tile (and every split's k range) is whole and aligned.
bool tiles_exact(const GemmArgs &a, int bm, int bn, int bk) {
    return a.M % bm == 0 && a.N % bn == 0 && a.K % bk == 0 && a.k_per_split % bk == 0 &&
           a.a_vec_ok && a.b_vec_ok;
}

// The FP32 256 x 128 tile (one block per CU, 64 x 128 accumulators per wave): plain products with a
// k-contiguous A (X.W and X.W^T) on whole tiles and whole k-tiles.
// The FP32 64 x 32 tile: plain products (any layout).
bool f32_6432_applicable(const GemmArgs &a) {
    return !a.dual && !a.xent_stats && !a.a_kscale && a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL;
}

bool f32_256_applicable(bool ta, const GemmArgs &a) {
    return !ta && !a.dual && !a.xent_stats && !a.a_kscale && !a.swiglu_bwd && !a.rope_table &&
           a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL && tiles_exact(a, 256, 128, ET<float>::BK);
}


// The direct-to-LDS kernel takes whole tiles without epilogue masks or k limits, an even number of
// k-tiles per split, and 32-bit buffer offsets: a k-contiguous operand's 256 rows, or an
// mn-contiguous operand's k range, within 2 GiB.
// bn: the output tile width, 256 or 128 (the SwiGLU form's 256 x 128 output tile is given as 256).
bool dtl_applicable(bool ta, bool tb, const GemmArgs &a, int bn = 256) {
    auto fits = [&](bool kcontig, int64_t ld) {
        return kcontig ? ld * 2 * 256 < (1ll << 31) : a.k_per_split * ld * 2 < (1ll << 31);
    };
    if (bn != 256 && (bn != 128 || a.dual)) return false;
    return a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL && !a.swiglu_bwd && !a.xent_stats && !a.a_kscale &&
           (!a.dual || (!ta && tb)) && tiles_exact(a, 256, a.dual ? 128 : bn, ET<uint16_t>::BK) &&
           a.k_per_split % (2 * ET<uint16_t>::BK) == 0 && a.K % (2 * ET<uint16_t>::BK) == 0 &&
           fits(!ta, a.lda) && fits(tb, a.ldb) && a.K * 2 < (1ll << 31);
}

// The 128 x 128 direct-to-LDS kernel: whole tiles, any number of 64-wide k-tiles per split, and
// 32-bit buffer offsets (a k-contiguous operand's 128 rows, or an mn-contiguous one's k range, within
// 2 GiB).
bool dtl128_applicable(bool ta, bool tb, const GemmArgs &a) {
    auto fits = [&](bool kcontig, int64_t ld) {
        return kcontig ? ld * 2 * 128 < (1ll << 31) : a.k_per_split * ld * 2 < (1ll << 31);
    };
    return !a.dual && a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL && !a.swiglu_bwd && !a.xent_stats &&
           !a.a_kscale && tiles_exact(a, 128, 128, ET<uint16_t>::BK) && a.k_per_split % ET<uint16_t>::BK == 0 &&
           fits(!ta, a.lda) && fits(tb, a.ldb) && a.K * 2 < (1ll << 31);
}

hipError_t launch_bf16_dtl128(bool ta, bool tb, const GemmArgs &a, dim3 grid, hipStream_t s) {
    if (!ta && tb) hipLaunchKernelGGL((gemm_bf16_dtl128<false, true>), grid, dim3(NTHREADS), 0, s, a);
    else if (!ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl128<false, false>), grid, dim3(NTHREADS), 0, s, a);
    else if (ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl128<true, false>), grid, dim3(NTHREADS), 0, s, a);
    else hipLaunchKernelGGL((gemm_bf16_dtl128<true, true>), grid, dim3(NTHREADS), 0, s, a);
    return hipGetLastError();
}

hipError_t launch_bf16_256(bool ta, bool tb, int bn, const GemmArgs &a, dim3 grid, hipStream_t s) {
    if (bn == 128) {  // the planner offers 256 x 128 only where the direct-to-LDS kernel applies
        if (!dtl_applicable(ta, tb, a, 128)) return hipErrorInvalidConfiguration;
        if (!ta && tb) hipLaunchKernelGGL((gemm_bf16_dtl<false, true, false, 2>), grid, dim3(NTHREADS), 0, s, a);
        else if (!ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl<false, false, false, 2>), grid, dim3(NTHREADS), 0, s, a);
        else if (ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl<true, false, false, 2>), grid, dim3(NTHREADS), 0, s, a);
        else hipLaunchKernelGGL((gemm_bf16_dtl<true, true, false, 2>), grid, dim3(NTHREADS), 0, s, a);
        return hipGetLastError();
    }
    if (dtl_applicable(ta, tb, a)) {
        if (a.dual) hipLaunchKernelGGL((gemm_bf16_dtl<false, true, true>), grid, dim3(NTHREADS), 0, s, a);
        else if (!ta && tb) hipLaunchKernelGGL((gemm_bf16_dtl<false, true>), grid, dim3(NTHREADS), 0, s, a);
        else if (!ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl<false, false>), grid, dim3(NTHREADS), 0, s, a);
        else if (ta && !tb) hipLaunchKernelGGL((gemm_bf16_dtl<true, false>), grid, dim3(NTHREADS), 0, s, a);
        else hipLaunchKernelGGL((gemm_bf16_dtl<true, true>), grid, dim3(NTHREADS), 0, s, a);
        return hipGetLastError();
    }
    if (tiles_exact(a, 256, a.dual ? 128 : 256, ET<uint16_t>::BK))
        launch_bf16_256_e<false>(ta, tb, a, grid, s);
    else
        launch_bf16_256_e<true>(ta, tb, a, grid, s);
    return hipGetLastError();
}

// The 64x64 FP32 tile has register room for a second staging set: its loads run two k-tiles
// ahead (measured 2-18% faster on the TINY step's small GEMMs; the 128x128 tile measured slower
// with it and keeps one).
template <typename T, bool TA, bool TB, bool DUAL, int LM, bool KS = false>
void launch_cfg_lm(const TileCfg &cfg, const GemmArgs &a, dim3 grid, hipStream_t s) {
    constexpr int PF64 = sizeof(T) == 4 ? 2 : 1;
    if constexpr (sizeof(T) == 4 && !TA && !DUAL && !KS && LM == LOAD_EXACT) {
        if (cfg.bm == 256) {
            hipLaunchKernelGGL((gemm_mfma<T, TA, TB, 256, 128, 2, 2, DUAL, LM, KS, 1>), grid, dim3(NTHREADS), 0, s, a);
            return;
        }
    }
    if constexpr (sizeof(T) == 4 && !DUAL && !KS) {
        if (cfg.bm == 64 && cfg.bn == 32) {
            hipLaunchKernelGGL((gemm_mfma<T, TA, TB, 64, 32, 2, 2, DUAL, LM, KS, PF64>), grid, dim3(NTHREADS), 0, s, a);
            return;
        }
    }
    if (cfg.bm == 128)
        hipLaunchKernelGGL((gemm_mfma<T, TA, TB, 128, 128, 2, 2, DUAL, LM, KS>), grid, dim3(NTHREADS), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_mfma<T, TA, TB, 64, 64, 2, 2, DUAL, LM, KS, PF64>), grid, dim3(NTHREADS), 0, s, a);
}

// Branch-free masked loads need aligned 16-byte vectors that never straddle an edge.
template <typename T>
bool vectors_exact(const GemmArgs &a, bool ta, bool tb) {
    constexpr int VEC = ET<T>::VEC;
    return a.a_vec_ok && a.b_vec_ok && a.K % VEC == 0 && (!ta || a.M % VEC == 0) && (tb || a.N % VEC == 0);
}

// LOAD_RSRC (FP32): 16-byte vectors as LOAD_MASKED, no k tail inside a k-contiguous operand's rows
// (K a multiple of the k-tile), and each operand's valid bytes within a 32-bit range.
bool rsrc_ok(const GemmArgs &a, bool ta, bool tb) {
    const bool kcontig = !ta || tb;
    return vectors_exact<float>(a, ta, tb) && (!kcontig || a.K % ET<float>::BK == 0) &&
           (ta ? a.K : a.M) * a.lda * 4 < (1ll << 31) && (tb ? a.N : a.K) * a.ldb * 4 < (1ll << 31);
}

// The load mode of a plain tile: exact, buffer-descriptor (FP32), masked or checked.
template <typename T>
int load_mode_for(const GemmArgs &a, bool ta, bool tb, int bm, int bn) {
    int mode = tiles_exact(a, bm, bn, ET<T>::BK)                        ? LOAD_EXACT
               : sizeof(T) == 4 && rsrc_ok(a, ta, tb)                     ? LOAD_RSRC
               : vectors_exact<T>(a, ta, tb)                              ? LOAD_MASKED
                                                                          : LOAD_CHECKED;
#ifdef IT_TUNING
    // Planner sweeps only: IT_LOAD_MODE=masked|rsrc forces one of the two where both apply.
    if (const char *env = std::getenv("IT_LOAD_MODE")) {
        const std::string m(env);
        if (sizeof(T) == 4 && m == "rsrc" && rsrc_ok(a, ta, tb)) mode = LOAD_RSRC;
        if (m == "masked" && mode == LOAD_RSRC) mode = LOAD_MASKED;
    }
#endif
    return mode;
}

template <typename T, bool TA, bool TB, bool DUAL>
hipError_t launch_cfg(const TileCfg &cfg, const GemmArgs &a, dim3 grid, hipStream_t s) {
    const int mode = DUAL ? (tiles_exact(a, cfg.bm, cfg.bn / 2, ET<T>::BK) ? LOAD_EXACT
                             : vectors_exact<T>(a, TA, TB)                  ? LOAD_MASKED
                                                                            : LOAD_CHECKED)
                          : load_mode_for<T>(a, TA, TB, cfg.bm, cfg.bn);
    if (mode == LOAD_EXACT)
        launch_cfg_lm<T, TA, TB, DUAL, LOAD_EXACT>(cfg, a, grid, s);
    else if (mode == LOAD_MASKED)
        launch_cfg_lm<T, TA, TB, DUAL, LOAD_MASKED>(cfg, a, grid, s);
    else if constexpr (sizeof(T) == 4 && !DUAL) {
        if (mode == LOAD_RSRC)
            launch_cfg_lm<T, TA, TB, DUAL, LOAD_RSRC>(cfg, a, grid, s);
        else
            launch_cfg_lm<T, TA, TB, DUAL, LOAD_CHECKED>(cfg, a, grid, s);
    } else {
        launch_cfg_lm<T, TA, TB, DUAL, LOAD_CHECKED>(cfg, a, grid, s);
    }
    return hipGetLastError();
}

// Cross-entropy gradient operand (FP32, B not transposed; checked by the caller).
template <bool TA, int LM>
void launch_xent_lm(const TileCfg &cfg, const GemmArgs &a, dim3 grid, hipStream_t s) {
    if (cfg.bm == 128)
        hipLaunchKernelGGL((gemm_mfma<float, TA, false, 128, 128, 2, 2, false, LM, false, 1, true>), grid,
                           dim3(NTHREADS), 0, s, a);
    else
        hipLaunchKernelGGL((gemm_mfma<float, TA, false, 64, 64, 2, 2, false, LM, false, 2, true>), grid,
                           dim3(NTHREADS), 0, s, a);
}

template <bool TA>
hipError_t launch_xent(const TileCfg &cfg, const GemmArgs &a, dim3 grid, hipStream_t s) {
    if (tiles_exact(a, cfg.bm, cfg.bn, ET<float>::BK))
        launch_xent_lm<TA, LOAD_EXACT>(cfg, a, grid, s);
    else if (vectors_exact<float>(a, TA, false))
        launch_xent_lm<TA, LOAD_MASKED>(cfg, a, grid, s);
    else
        launch_xent_lm<TA, LOAD_CHECKED>(cfg, a, grid, s);
    return hipGetLastError();
}

template <typename T>
hipError_t launch_typed(bool ta, bool tb, bool dual, const TileCfg &cfg, const GemmArgs &a, dim3 grid,
                        hipStream_t s) {
    if constexpr (sizeof(T) == 4) {
        if (a.xent_stats) return ta ? launch_xent<true>(cfg, a, grid, s) : launch_xent<false>(cfg, a, grid, s);
        if (a.a_kscale) {  // fused RMSNorm + projection: X.W^T only (checked by the caller)
            if (vectors_exact<T>(a, false, true))
                launch_cfg_lm<T, false, true, false, LOAD_MASKED, true>(cfg, a, grid, s);
            else
                launch_cfg_lm<T, false, true, false, LOAD_CHECKED, true>(cfg, a, grid, s);
            return hipGetLastError();
        }
    }
    if (dual) return launch_cfg<T, false, true, true>(cfg, a, grid, s);
    if (!ta && !tb) return launch_cfg<T, false, false, false>(cfg, a, grid, s);
    if (!ta && tb) return launch_cfg<T, false, true, false>(cfg, a, grid, s);
    if (ta && !tb) return launch_cfg<T, true, false, false>(cfg, a, grid, s);
    return launch_cfg<T, true, true, false>(cfg, a, grid, s);
}

int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

struct Plan {
    int bm, bn, splits;
    int64_t k_per_split;  // 0: K / splits rounded up to the k-tile
};

// Picks the tile shape and split-K factor with a cost model fitted to MI355X timings of these
// kernels: every tile / split choice on the TINY and medium step shapes, the square sweep and the
// decode shapes. The efficiencies were refitted after later kernel changes, on sweeps that time
// each plan with caches flushed (and, for FP32, also warm):
//   * BF16, 32 shapes: the picks take 0.2% longer in total than the fastest measured plans
//     (3.3% with the first fit, whose 128x128 efficiency kept the medium step's long-K data
//     gradients off the 256x256 tile);
//   * FP32, the 14 plain TINY step shapes: 0.6% longer (2.9% with the first fit, which put the
//     LM-head GEMMs on 128x128 tiles where the prefetching 64x64 tile is now 5-8% faster).
// The model:
//   * a CU runs up to `occ` blocks at once, sharing its MFMA rate (a lone block where two could
//     run reaches 90% of the tile's efficiency);
//   * each round of blocks pays a fixed prologue/epilogue cost;
//   * a k-step costs the larger of its MFMA time (at the tile's steady-state efficiency, times
//     the blocks sharing the CU) and a memory-latency floor: with one tile of prefetch, a block
//     waits on its loads when a k-step has too little work to cover them (long-K, small-M/N
//     weight gradients), which is what split-K fixes by running more blocks at once;
//   * split-K adds its partial-sum traffic and a reduction launch.
// Estimated seconds, lowest wins.
// est (optional): the chosen plan's estimated seconds.
Plan choose_plan(const GemmArgs &a, bool bf16, int64_t cus, bool ta, bool tb, double *est = nullptr) {
    struct Cand {
        int b, bn, occ;  // b x bn tiles (bn 0: square)
        double eff;
    };
    // FP32 256 x 128 (one block per CU): fitted on the LM-head data gradient [4096,256,16384] (eight
    // splits: 274 us against 291-302 us for the best 64 x 64 plans), with a per-round cost that
    // covers its 128 KB epilogue (the LM-head forward, 8 rounds of 8 k-steps: 361 us). Offered for
    // long k ranges only (32 k-steps per split or more), where it measured faster.
    // FP32 64 x 32 (plain products): two blocks per CU where the 64 x 64 tiles leave one, e.g. the
    // TINY step's [4096, 256, K] GEMMs (3-7% faster at K 256-1376); the model prices it at the 64 x 64
    // tile's efficiency.
    const Cand f32c[] = {{128, 0, 2, 0.50}, {64, 0, 4, 0.60}, {256, 128, 1, 0.87}, {64, 32, 4, 0.60}};
    constexpr double F32_256_ROUND = 14e-6;
    constexpr int64_t F32_256_MIN_KSTEPS = 32;
    // 256 x 128 exists only as the direct-to-LDS kernel (eff 0: skipped where that does not apply).
    // The register-staged 64 x 64 BF16 tile transposes [k][mn] operands in registers on the way to
    // LDS: measured (1536^3, 2048^3) about 0.24 of the per-CU rate with no transpose (NT), 0.20 with
    // B transposed (NN) and 0.15-0.19 with A transposed.
    const double e64 = ta ? 0.15 : tb ? 0.24 : 0.20;
    const Cand b16c[] = {{256, 0, 1, 0.40}, {256, 128, 1, 0.0}, {128, 0, 2, 0.20}, {64, 0, 4, e64}};
    // The direct-to-LDS kernel (whole tiles, an even number of k-tiles per split): 256 x 256, and
    // 256 x 128, whose waves read 50% more LDS per MFMA (two transposed reads per fragment of a
    // transposed A: lower still), and whose third stage lowers the memory-latency floor.
    constexpr double DTL_EFF = 0.53, DTL_HALF_FLOOR = 0.85e-6;
    // The 128 x 128 direct-to-LDS tile (four stages: three k-tiles of loads in flight), the same in
    // every layout: 1024^3 11.5-11.8 us, 1280^3 13.9-14.1, 1536^3 15.9-16.3, 2048^3 (one tile per
    // CU) 22.0-22.8 against 32-35 us for the 256 x 128 plans; 0.38 of the per-CU rate with the
    // 3 us round cost fits them within 3%.
    constexpr double DTL128_EFF = 0.38;
    constexpr double DTL128_FLOOR = 0.35e-6;
    const double DTL_HALF_EFF = ta ? 0.42 : 0.52;
    const Cand *cands = bf16 ? b16c : f32c;
    constexpr int ncand = 4;
    const int bk = bf16 ? ET<uint16_t>::BK : ET<float>::BK;
    const double cu_peak = (bf16 ? 2.5e15 : 157.3e12) / 256.0;  // FLOP/s per CU
    const double round_overhead = 3e-6, reduce_launch = 4e-6, partial_bw = 4e12;
    const double step_floor = bf16 ? 1.0e-6 : 0.5e-6;
    constexpr double F64_FLOOR_NT = 0.4e-6, F64_FLOOR_NN = 0.6e-6, F64_FLOOR_TA = 1.05e-6;
    const bool can_split = !a.dual && a.causal == CAUSAL_NONE && a.kmode == KMODE_FULL && !a.no_split;
    Plan best{64, 64, 1, 0};
    double best_t = 1e30;
    int64_t best_blocks = 0;
    for (int c = 0; c < ncand; ++c) {
        const Cand &cd = cands[c];
        if (cd.bn && a.dual) continue;
        // A dual (SwiGLU) tile covers b x b/2 outputs: its b B-tile rows are gate and up halves.
        const int bn = a.dual ? cd.b / 2 : cd.bn ? cd.bn : cd.b;
        const int64_t tiles = cdiv(a.M, cd.b) * cdiv(a.N, bn) * a.batch;
        if (cd.b == 256) {
            const double fill = (double)a.M * a.N * a.batch / ((double)tiles * 256.0 * bn);
            if (fill < 0.7) continue;
        }
        // BF16 tries every split count (a multiple of 128 per split, as the direct-to-LDS kernel
        // needs: 5 splits fill 240 CUs with a 48-tile weight gradient where 4 fill 192); FP32
        // powers of two.
        for (int s = 1; s <= 32; s = bf16 ? s + 1 : 2 * s) {
            if (s > 1 && !can_split) break;
            const int64_t kunit = bf16 ? 2 * bk : bk;
            const int64_t kps = cdiv(cdiv(a.K, s), kunit) * kunit;
            if (s > 1 && kps < 4 * bk) break;
            const int64_t splits = s > 1 ? cdiv(a.K, kps) : 1;
            const int64_t blocks = tiles * splits;
            const int64_t per_cu = cdiv(blocks, cus);
            // The 128 x 128 BF16 tile runs on the direct-to-LDS kernel where it applies (one block
            // per CU: its stages take 128 KB of LDS).
            GemmArgs d = a;
            d.k_per_split = kps;
            const bool d128 = bf16 && cd.b == 128 && dtl128_applicable(ta, tb, d);
            const int occ = d128 ? 1 : cd.occ;
            const int64_t conc = std::min<int64_t>(per_cu, occ);
            const int64_t rounds = cdiv(per_cu, occ);
            const int64_t ksteps = std::max<int64_t>(1, cdiv(kps, bk));
            // A lone block on a CU whose tile could run two at once hides less latency.
            double eff = conc == 1 && occ > 1 ? 0.9 * cd.eff : cd.eff;
            double floor = bf16 && cd.bn == 128 ? DTL_HALF_FLOOR : step_floor;
            double ro = round_overhead;
            if (!bf16 && cd.b == 256) {
                if (!f32_256_applicable(ta, d) || ksteps < F32_256_MIN_KSTEPS) continue;
                ro = F32_256_ROUND;
            }
            if (!bf16 && cd.bn == 32 && !f32_6432_applicable(d)) continue;
            // The register-staged BF16 64 x 64 tile with one block per CU (1024^3: 16 k-steps on 256
            // CUs) measured 0.4 / 0.6 / 0.85 us per k-step for NT / NN / transposed A (9.6 / 13.0 /
            // 16.4 us), not the 1 us floor of the larger tiles' loads.
            if (bf16 && cd.b == 64 && !cd.bn) floor = ta ? F64_FLOOR_TA : tb ? F64_FLOOR_NT : F64_FLOOR_NN;
            if (bf16 && cd.b == 256 && dtl_applicable(ta, tb, d, a.dual ? 256 : bn))
                eff = bn == 128 && !a.dual ? DTL_HALF_EFF : DTL_EFF;
            if (d128) {
                eff = DTL128_EFF;
                floor = DTL128_FLOOR;
            }
            if (eff <= 0.0) continue;
            const double step = (a.dual ? 4.0 : 2.0) * cd.b * bn * bk / (cu_peak * eff);
            double t = rounds * (ro + ksteps * std::max(conc * step, floor));
            if (splits > 1) t += 2.0 * splits * a.M * a.N * a.batch * 4.0 / partial_bw + reduce_launch;
            // Near ties (3%) keep the earlier, larger and less split plan, except that between two
            // unsplit plans the one with more blocks wins (more loads in flight per k-step); the
            // FP32 64 x 32 tile has to win outright.
            const bool better = t < best_t * 0.97;
            const bool tie_more_blocks = t < best_t * 1.03 && splits == 1 && best.splits == 1 &&
                                         blocks > best_blocks && cd.bn != 32;
            if (better || tie_more_blocks) {
                best_t = better ? t : std::min(t, best_t);
                best = Plan{cd.b, bn, (int)splits, splits > 1 ? kps : 0};
                best_blocks = blocks;
            }
        }
    }
    if (est) *est = best_t;
    return best;
}

}  // namespace

it_status launch_splitk_reduce(hipStream_t s, const GemmArgs &a) {
    const int64_t total = a.batch * a.M * a.N;
    if (a.N % 4 == 0) {
        const int64_t blocks = std::min<int64_t>(cdiv(total / 4, 256), 65536);
        hipLaunchKernelGGL(splitk_reduce4, dim3((unsigned)blocks), dim3(256), 0, s, a);
        IT_HIP_TRY(hipGetLastError());
        return IT_OK;
    }
    const int64_t blocks = std::min<int64_t>(cdiv(total, 256), 65536);
    hipLaunchKernelGGL(splitk_reduce, dim3((unsigned)blocks), dim3(256), 0, s, a);
    IT_HIP_TRY(hipGetLastError());
    return IT_OK;
}

it_status launch_gemm(it_context *ctx, it_dtype dtype_in, bool transA, bool transB, GemmArgs a,
                      const char *profile_tag) {
    const bool bf16 = dtype_in == IT_BF16;
    if (gemv_applicable(a, bf16, transA, transB)) {
        std::string key;
        hipEvent_t ev = nullptr;
        if (ctx->profiling) {
            char buf[160];
            std::snprintf(buf, sizeof(buf), "gemv_bf16_NT|%s[%lld,%lld,%lld]x%lld s1", profile_tag ? profile_tag : "",
                          (long long)a.M, (long long)a.N, (long long)a.K, (long long)a.batch);
            key = buf;
            profile_begin(ctx, key, &ev);
        }
        const it_status st = launch_gemv(ctx->stream, a);
        if (ctx->profiling) profile_end(ctx, key, ev);
        return st;
    }
    if (gemv_kn_applicable(a, bf16, transA, transB)) {
        int ks = gemv_kn_splits(a, transA);
#ifdef IT_TUNING
        if (const char *env = std::getenv("IT_GEMV_KS"))
            ks = std::max(gemv_kn_min_splits(a, transA), std::min(32, std::max(1, std::atoi(env))));
#endif
        a.k_per_split = cdiv(cdiv(a.K, ks), 128) * 128;
        a.splits = (int)cdiv(a.K, a.k_per_split);
        int *counters = nullptr;
        if (a.splits > 1) {
            void *ws = nullptr;
            it_status st = ensure_scratch(ctx, (size_t)a.splits * a.batch * a.M * a.N * sizeof(float), &ws);
            if (st != IT_OK) return st;
            a.partial = (float *)ws;
            st = ensure_counters(ctx, &counters);
            if (st != IT_OK) return st;
        }
        std::string key;
        hipEvent_t ev = nullptr;
        if (ctx->profiling) {
            char buf[160];
            std::snprintf(buf, sizeof(buf), "gemv_bf16_%cN|%s[%lld,%lld,%lld]x%lld s%d", transA ? 'T' : 'N',
                          profile_tag ? profile_tag : "", (long long)a.M, (long long)a.N, (long long)a.K,
                          (long long)a.batch, a.splits);
            key = buf;
            profile_begin(ctx, key, &ev);
        }
        const it_status st = launch_gemv_kn(ctx->stream, transA, a, counters);
        if (ctx->profiling) profile_end(ctx, key, ev);
        return st;
    }
    const int bk = bf16 ? ET<uint16_t>::BK : ET<float>::BK;
    const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    Plan plan = choose_plan(a, bf16, cus, transA, transB);
#ifdef IT_TUNING
    // Planner sweeps only (a tuning build): IT_PLAN="tile,splits[,width]" forces the plan.
    if (const char *env = std::getenv("IT_PLAN")) {
        int b = 0, sp = 0, w = 0;
        const int n = std::sscanf(env, "%d,%d,%d", &b, &sp, &w);
        if (n >= 2) plan = Plan{b, a.dual ? b / 2 : n == 3 ? w : b, sp, bf16 && sp > 1 ? cdiv(cdiv(a.K, sp), 128) * 128 : 0};
    }
#endif
    TileCfg cfg{plan.bm, plan.bn};
    int splits = plan.splits;
    a.tiles_m = (int)cdiv(a.M, cfg.bm);
    a.tiles_n = (int)cdiv(a.N, cfg.bn);
    int64_t kps = plan.k_per_split;
    if (kps <= 0) kps = cdiv(cdiv(a.K, splits), bk) * bk;
    if (kps == 0) kps = bk;
    splits = (int)std::max<int64_t>(1, cdiv(a.K, kps));
    a.k_per_split = kps;
    a.splits = splits;
    // The FP32 256 x 128 tile covers plain GEMMs with a k-contiguous A on whole tiles only (the
    // planner offers it for nothing else).
    if (!bf16 && cfg.bm == 256 && (cfg.bn != 128 || !f32_256_applicable(transA, a)))
        return fail(IT_ERR_INVALID, "it_gemm: no FP32 256-row tile for this product");
    if (!bf16 && !a.dual && cfg.bn == 32 && (cfg.bm != 64 || !f32_6432_applicable(a)))
        return fail(IT_ERR_INVALID, "it_gemm: no FP32 64 x 32 tile for this product");
    if (splits > 1) {
        void *ws = nullptr;
        it_status st = ensure_scratch(ctx, (size_t)splits * a.batch * a.M * a.N * sizeof(float), &ws);
        if (st != IT_OK) return st;
        a.partial = (float *)ws;
    }
    const bool dtl128 = bf16 && cfg.bm == 128 && cfg.bn == 128 && dtl128_applicable(transA, transB, a);
    const bool dtl = dtl128 || (bf16 && cfg.bm == 256 && dtl_applicable(transA, transB, a, a.dual ? 256 : cfg.bn));

    const int64_t gx = (int64_t)a.tiles_m * a.tiles_n;
    const int64_t gy = a.batch * splits;
    if (gx > 0x7fffffff || gy > 65535)
        return fail(IT_ERR_DIMS, "it_gemm: grid too large (tiles " + std::to_string(gx) +
                                     ", batch*splits " + std::to_string(gy) + ")");
    dim3 grid((unsigned)gx, (unsigned)gy);

    std::string key;
    hipEvent_t ev = nullptr;
    if (ctx->profiling) {
        char buf[192];
        std::snprintf(buf, sizeof(buf), "gemm_%s_%c%c_%dx%d%s%s%s%s|%s[%lld,%lld,%lld]x%lld s%d",
                      bf16 ? "bf16" : "f32", transA ? 'T' : 'N', transB ? 'T' : 'N', cfg.bm, cfg.bn,
                      dtl ? "_dtl" : "",
                      a.dual ? "_swiglu" : "", a.causal || a.kmode ? "_causal" : "", a.a_kscale ? "_rmsnorm" : a.xent_stats ? "_xent" : "",
                      profile_tag ? profile_tag : "", (long long)a.M, (long long)a.N,
                      (long long)a.K, (long long)a.batch, splits);
        key = buf;
        profile_begin(ctx, key, &ev);
    }
    hipError_t e = bf16 && cfg.bm == 256 ? launch_bf16_256(transA, transB, a.dual ? 256 : cfg.bn, a, grid, ctx->stream)
                   : dtl128      ? launch_bf16_dtl128(transA, transB, a, grid, ctx->stream)
                   : bf16        ? launch_typed<uint16_t>(transA, transB, a.dual, cfg, a, grid, ctx->stream)
                                 : launch_typed<float>(transA, transB, a.dual, cfg, a, grid, ctx->stream);
    if (e != hipSuccess) return fail_hip(e, "gemm_mfma launch");
    if (splits > 1) {
        it_status st = launch_splitk_reduce(ctx->stream, a);
        if (st != IT_OK) return st;
    }
    if (ctx->profiling) profile_end(ctx, key, ev);
    return IT_OK;
}


namespace {

// Prepares a for a one-split 256 x 256 direct-to-LDS block in a group; false if it does not qualify.
bool group_256(GemmArgs &a, bool bf16, bool ta, bool tb) {
    a.splits = 1;
    a.k_per_split = a.K;
    a.tiles_m = (int)cdiv(a.M, 256);
    a.tiles_n = (int)cdiv(a.N, 256);
    return bf16 && a.batch == 1 && !a.dual && a.K > 0 && dtl_applicable(ta, tb, a, 256) &&
           !gemv_applicable(a, bf16, ta, tb) && !gemv_kn_applicable(a, bf16, ta, tb);
}

// The group's XCD schedule (GemmGroupArgs): the blocks of every problem (tiles x splits, in call
// and split order) cut into eight equal shares, one per XCD. Returns the grid size, or 0 when the
// schedule does not fit the table (the caller then launches the calls separately).
int xcd_schedule(GemmGroupArgs &grp) {
    int64_t total = 0;
    for (int i = 0; i < grp.count; ++i) {
        const int64_t tiles = (int64_t)grp.g[i].tiles_m * grp.g[i].tiles_n;
        if (tiles > 65535 || grp.g[i].splits > 255) return 0;
        total += tiles * grp.g[i].splits;
    }
    const int64_t per = cdiv(total, 8);
    if (total == 0 || per > 65535) return 0;
    int x = 0, nch = 0;
    int64_t filled = 0;
    grp.xstart[0] = 0;
    for (int i = 0; i < grp.count; ++i) {
        const int64_t tiles = (int64_t)grp.g[i].tiles_m * grp.g[i].tiles_n;
        for (int sp = 0; sp < grp.g[i].splits; ++sp)
            for (int64_t t = 0; t < tiles;) {
                if (filled == per) {  // this XCD's share is full: the next one starts
                    if (x == 7) return 0;
                    grp.xn[x++] = (uint16_t)per;
                    grp.xstart[x] = (uint16_t)nch;
                    filled = 0;
                }
                if (nch == GROUP_CHUNKS) return 0;
                grp.chunk[nch++] = GroupChunk{(uint16_t)filled, (uint8_t)i, (uint8_t)sp, (uint16_t)t, 0};
                const int64_t take = std::min(tiles - t, per - filled);
                t += take;
                filled += take;
            }
    }
    grp.xn[x] = (uint16_t)filled;
    for (int y = x + 1; y < 8; ++y) {
        grp.xn[y] = 0;
        grp.xstart[y] = (uint16_t)nch;
    }
    grp.xstart[8] = (uint16_t)nch;
    return (int)(8 * per);
}

// The planner's pricing of a direct-to-LDS block that runs `k` of K: k-steps at the tile's rate or
// the latency floor.
double dtl_block_time(int64_t k, int bn, bool ta) {
    const double cu_peak = 2.5e15 / 256.0;
    const double eff = bn == 256 ? 0.53 : ta ? 0.42 : 0.52;
    const double step = 2.0 * 256 * bn * 64 / (cu_peak * eff);
    return cdiv(k, 64) * std::max(step, bn == 256 ? 1.0e-6 : 0.85e-6);
}

it_status launch_group_kernel(it_context *ctx, const GemmGroupArgs &grp, int blocks, bool ta, bool tb,
                              const std::string &key) {
    hipEvent_t ev = nullptr;
    if (ctx->profiling) profile_begin(ctx, key, &ev);
    const dim3 grid((unsigned)blocks);
    if (!ta && tb) {
        hipLaunchKernelGGL((gemm_bf16_dtl_group<false, true>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
    } else if (!ta && !tb) {
        hipLaunchKernelGGL((gemm_bf16_dtl_group<false, false>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
    } else if (ta && !tb) {
        hipLaunchKernelGGL((gemm_bf16_dtl_group<true, false>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
    } else {
        hipLaunchKernelGGL((gemm_bf16_dtl_group<true, true>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
    }
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return fail_hip(e, "gemm group launch");
    if (ctx->profiling) profile_end(ctx, key, ev);
    return IT_OK;
}

std::string group_key(const char *form, const GemmArgs *args, int count, const char *tag) {
    std::string key = std::string("gemm_bf16_") + form + "|" + (tag ? tag : "");
    for (int i = 0; i < count; ++i)
        key += (i ? "+[" : "[") + std::to_string(args[i].M) + "," + std::to_string(args[i].N) + "," +
               std::to_string(args[i].K) + "]";
    return key + "x1 s1";
}

// FP32 calls of one layout: one gemm_f32_group launch (64 x 64 tiles, one split count for the
// group; each tile's last split block adds the partial sums) where the planner's model prices it
// below the separate plans; false if they do not qualify or do not pay (nothing launched then).
bool launch_f32_group(it_context *ctx, bool ta, bool tb, GemmArgs *args, int count, const char *tag,
                      it_status *status) {
    constexpr int bk = ET<float>::BK;
    const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    if (count < 2) return false;
    double separate = 0.0;
    for (int i = 0; i < count; ++i) {
        const GemmArgs &a = args[i];
        if (a.batch != 1 || a.dual || a.causal != CAUSAL_NONE || a.kmode != KMODE_FULL || a.swiglu_bwd ||
            a.xent_stats || a.a_kscale || a.K <= 0 || a.N % 4 != 0 || a.no_split || gemv_applicable(a, false, ta, tb))
            return false;
        double t = 0.0;
        const Plan pl = choose_plan(a, false, cus, ta, tb, &t);
        if (pl.bm != 64) return false;  // the group runs 64 x 64 tiles only
        separate += t;
    }
    // The planner's model of the group at one split count s: 64 x 64 tiles, up to 4 blocks per CU.
    // The XCD schedule takes at most count * s + 7 chunks (a chunk per GEMM and split, plus one
    // more where an XCD's share ends inside one), so s stays where that fits the table.
    const double cu_peak = 157.3e12 / 256.0, eff0 = 0.60;
    double best_t = 1e30;
    int best_s = 0;
    for (int s = 1; s <= 32 && count * s + 7 <= GROUP_CHUNKS; ++s) {
        int64_t blocks = 0, ksteps = 0;
        double traffic = 0.0;
        bool ok = true;
        for (int i = 0; i < count && ok; ++i) {
            const GemmArgs &a = args[i];
            const int64_t kps = cdiv(cdiv(a.K, s), bk) * bk;
            ok = s == 1 || kps >= 4 * bk;
            const int64_t splits = s > 1 ? cdiv(a.K, kps) : 1;
            blocks += cdiv(a.M, 64) * cdiv(a.N, 64) * splits;
            ksteps = std::max(ksteps, cdiv(kps, bk));
            if (splits > 1) traffic += 2.0 * splits * a.M * a.N * 4.0;
        }
        if (!ok) break;
        const int64_t per_cu = cdiv(blocks, cus), conc = std::min<int64_t>(per_cu, 4), rounds = cdiv(per_cu, 4);
        const double eff = conc == 1 ? 0.9 * eff0 : eff0;
        const double step = 2.0 * 64 * 64 * bk / (cu_peak * eff);
        double t = rounds * (3e-6 + ksteps * std::max(conc * step, 0.5e-6));
        if (traffic > 0.0) t += traffic / 4e12 + 4e-6;  // partial sums out and back, the tiles' last-block sums
        if (t < best_t) {
            best_t = t;
            best_s = s;
        }
    }
#ifdef IT_TUNING
    // Planner sweeps only (a tuning build): IT_GROUP_SPLITS forces the group's split count.
    if (const char *env = std::getenv("IT_GROUP_SPLITS")) {
        best_s = std::max(1, std::min(32, std::atoi(env)));
        best_t = 0.0;
    }
#endif
    if (!best_s || best_t >= 0.97 * separate) return false;
    GemmGroupArgs grp{};
    grp.count = count;
    int64_t scratch = 0, tiles = 0;
    bool split_any = false, exact = true, masked = true, rsrc = true;
    for (int i = 0; i < count; ++i) {
        GemmArgs &a = grp.g[i];
        a = args[i];
        const int64_t kps = cdiv(cdiv(a.K, best_s), bk) * bk;
        a.splits = best_s > 1 ? (int)cdiv(a.K, kps) : 1;
        a.k_per_split = best_s > 1 ? kps : cdiv(a.K, bk) * bk;
        a.tiles_m = (int)cdiv(a.M, 64);
        a.tiles_n = (int)cdiv(a.N, 64);
        grp.cstart[i] = (int)tiles;
        tiles += (int64_t)a.tiles_m * a.tiles_n;
        if (a.splits > 1) {
            // the in-kernel sum addresses a problem's partials with 32-bit byte offsets
            if ((int64_t)a.splits * a.M * a.N * 4 >= (1ll << 31)) return false;
            split_any = true;
            scratch += (int64_t)a.splits * a.M * a.N;
        }
        exact = exact && tiles_exact(a, 64, 64, bk);
        masked = masked && vectors_exact<float>(a, ta, tb);
        rsrc = rsrc && load_mode_for<float>(a, ta, tb, 64, 64) != LOAD_MASKED && rsrc_ok(a, ta, tb);
    }
    if (tiles > COUNTERS) return false;
    grp.cstart[count] = (int)tiles;
    const int grid_blocks = xcd_schedule(grp);
    if (!grid_blocks) return false;
    if (split_any) {
        *status = ensure_counters(ctx, &grp.arrive);
        if (*status != IT_OK) return true;
    }
    if (scratch > 0) {
        void *ws = nullptr;
        *status = ensure_scratch(ctx, (size_t)scratch * sizeof(float), &ws);
        if (*status != IT_OK) return true;
        float *part = (float *)ws;
        for (int i = 0; i < count; ++i)
            if (grp.g[i].splits > 1) {
                grp.g[i].partial = part;
                part += (int64_t)grp.g[i].splits * grp.g[i].M * grp.g[i].N;
            }
    }
    std::string key;
    hipEvent_t ev = nullptr;
    if (ctx->profiling) {
        key = std::string("gemm_f32_") + (ta ? 'T' : 'N') + (tb ? 'T' : 'N') + "_64x64_group|" + (tag ? tag : "");
        for (int i = 0; i < count; ++i)
            key += (i ? "+[" : "[") + std::to_string(args[i].M) + "," + std::to_string(args[i].N) + "," +
                   std::to_string(args[i].K) + "]";
        key += "x1 s" + std::to_string(best_s);
        profile_begin(ctx, key, &ev);
    }
    const dim3 grid((unsigned)grid_blocks);
    auto go = [&](auto lm) {
        constexpr int LM = decltype(lm)::value;
        if (!ta && tb) hipLaunchKernelGGL((gemm_f32_group<false, true, LM>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
        else if (!ta && !tb) hipLaunchKernelGGL((gemm_f32_group<false, false, LM>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
        else if (ta && !tb) hipLaunchKernelGGL((gemm_f32_group<true, false, LM>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
        else hipLaunchKernelGGL((gemm_f32_group<true, true, LM>), grid, dim3(NTHREADS), 0, ctx->stream, grp);
    };
    if (exact) go(std::integral_constant<int, LOAD_EXACT>{});
    else if (rsrc) go(std::integral_constant<int, LOAD_RSRC>{});
    else if (masked) go(std::integral_constant<int, LOAD_MASKED>{});
    else go(std::integral_constant<int, LOAD_CHECKED>{});
    const hipError_t e = hipGetLastError();
    *status = e == hipSuccess ? IT_OK : fail_hip(e, "gemm group launch");
    if (ctx->profiling && *status == IT_OK) profile_end(ctx, key, ev);
    return true;
}

// Calls of one layout: one grouped launch where it pays, else launch_gemm each.
it_status launch_same_layout(it_context *ctx, it_dtype dtype_in, bool ta, bool tb, GemmArgs *args, int count,
                             const char *tag) {
    const bool bf16 = dtype_in == IT_BF16;
    if (!bf16) {
        it_status st = IT_OK;
        if (launch_f32_group(ctx, ta, tb, args, count, tag, &st)) return st;
    }
    const int64_t cus = ctx->num_cus > 0 ? ctx->num_cus : 256;
    bool fuse = count >= 2;
    int64_t blocks = 0, kmax = 0;
    double separate = 0.0;
    for (int i = 0; fuse && i < count; ++i) {
        GemmArgs a = args[i];
        fuse = group_256(a, bf16, ta, tb);
        blocks += (int64_t)a.tiles_m * a.tiles_n;
        double t = 0.0;
        choose_plan(args[i], bf16, cus, ta, tb, &t);
        separate += t;
        kmax = std::max(kmax, a.K);
    }
    // one round, every block over its whole K
    fuse = fuse && blocks <= cus && 3e-6 + dtl_block_time(kmax, 256, ta) < 0.97 * separate;
    if (!fuse) {
        for (int i = 0; i < count; ++i) {
            const it_status st = launch_gemm(ctx, dtype_in, ta, tb, args[i], tag);
            if (st != IT_OK) return st;
        }
        return IT_OK;
    }
    GemmGroupArgs grp{};
    grp.count = count;
    for (int i = 0; i < count; ++i) {
        grp.g[i] = args[i];
        group_256(grp.g[i], bf16, ta, tb);
    }
    const int grid = xcd_schedule(grp);
    if (!grid) {
        for (int i = 0; i < count; ++i) {
            const it_status st = launch_gemm(ctx, dtype_in, ta, tb, args[i], tag);
            if (st != IT_OK) return st;
        }
        return IT_OK;
    }
    const std::string form = std::string(1, ta ? 'T' : 'N') + (tb ? 'T' : 'N') + "_256x256_dtl_group";
    return launch_group_kernel(ctx, grp, grid, ta, tb,
                               ctx->profiling ? group_key(form.c_str(), grp.g, count, tag) : std::string());
}

}  // namespace

// Runs `count` independent GEMMs of one input dtype on ctx->stream (ta[i], tb[i]: their layouts),
// each run of consecutive calls of one layout as one gemm_bf16_dtl_group launch when they are BF16
// GEMMs of batch 1 that each take whole 256 x 256 direct-to-LDS tiles with one split and a plain
// epilogue, their tiles fit one round of CUs, and the planner's estimate for that round (every
// block running its whole K) beats the separate launches; else launch_gemm for each, as separate
// calls would run.
it_status launch_gemm_group(it_context *ctx, it_dtype dtype_in, const bool *ta, const bool *tb, GemmArgs *args,
                            int count, const char *profile_tag) {
    static_assert(sizeof(GemmGroupArgs) <= 4096, "kernel arguments");
    if (count <= 0) return IT_OK;
    if (count > GEMM_GROUP_MAX) return fail(IT_ERR_INVALID, "gemm group: more than 8 GEMMs");
    for (int i = 0; i < count;) {
        int j = i + 1;
        while (j < count && ta[j] == ta[i] && tb[j] == tb[i]) ++j;
        const it_status st = launch_same_layout(ctx, dtype_in, ta[i], tb[i], args + i, j - i, profile_tag);
        if (st != IT_OK) return st;
        i = j;
    }
    return IT_OK;
}

}  // namespace it
