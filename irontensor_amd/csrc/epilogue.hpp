// GEMM epilogue helpers shared by the tiled GEMM kernels, the split-K reduction and the decode
// kernels: the final value of an output element (alpha, beta, bias, causal mask, RoPE, the SwiGLU
// backward) or, for split-K, the raw partial sum; and the SwiGLU forward pair.
#pragma once

#include <cmath>

#include "internal.hpp"
#include "mfma.hpp"

namespace it {
namespace {

__device__ __forceinline__ float load_out(const void *C, int64_t idx, int bf16) {
    return bf16 ? bf16_to_f32(((const uint16_t *)C)[idx]) : ((const float *)C)[idx];
}

__device__ __forceinline__ void store_out(void *C, int64_t idx, float v, int bf16) {
    if (bf16)
        ((uint16_t *)C)[idx] = f32_to_bf16_rne(v);
    else
        ((float *)C)[idx] = v;
}

// Final value of one output element (alpha, beta, bias, causal), shared by the GEMM epilogue and
// the split-K reduction.
__device__ __forceinline__ float silu_grad(float go, float g, float u, float &du) {
    const float sig = sigmoid_fast(g);
    du = go * (g * sig);
    return go * u * (sig * (1.0f + g * (1.0f - sig)));
}

__device__ __forceinline__ void finish_store(const GemmArgs &p, void *C, int64_t idx, float acc,
                                             int64_t row, int64_t col) {
    float v = p.alpha * acc;
    if (p.swiglu_bwd) {  // dgate at idx, dup N columns later (C rows hold [dgate | dup])
        const int64_t gi = row * p.N + col;
        float du;
        const float dg = silu_grad(v, load_out(p.G, gi, p.out_bf16), load_out(p.U, gi, p.out_bf16), du);
        store_out(C, idx, dg, p.out_bf16);
        store_out(C, idx + p.N, du, p.out_bf16);
        return;
    }
    if (p.row_scale) v *= p.row_scale[row];
    if (p.beta != 0.f) v += p.beta * load_out(C, idx, p.out_bf16);
    if (p.has_bias) v += p.bias[col];
    if (p.causal != CAUSAL_NONE && col > row + p.causal_offset) v = -INFINITY;
    store_out(C, idx, v, p.out_bf16);
}

__device__ __forceinline__ float silu(float g) { return g * sigmoid_fast(g); }

// Final values of 4 consecutive output columns (the vector form of finish_store), or raw partial
// sums for split-K. Falls back to element stores at the right edge or for unaligned outputs.
template <bool EDGE, bool FINAL = false>
__device__ __forceinline__ void finish4(const GemmArgs &p, f32x4 v, int64_t row, int64_t col,
                                        int64_t coff, int64_t z) {
    if (EDGE && (row >= p.M || col >= p.N)) return;
    const bool full = !EDGE || col + 4 <= p.N;
    if (!FINAL && p.splits > 1) {
        float *dst = p.partial + (z * p.M + row) * p.N + col;
        if (full && p.N % 4 == 0) {
            *(f32x4 *)dst = v;
        } else {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e < p.N) dst[e] = v[e];
        }
        return;
    }
    const int64_t idx = coff + row * p.ldc + col;
    if (full && p.c_vec_ok) {
        v *= p.alpha;
        if (p.swiglu_bwd) {
            const int64_t gi = row * p.N + col;
            f32x4 g, u, dg, du;
            if (p.out_bf16) {
                const u32x2 gh = *(const u32x2 *)((const uint16_t *)p.G + gi), uh = *(const u32x2 *)((const uint16_t *)p.U + gi);
                g = f32x4{__uint_as_float(gh[0] << 16), __uint_as_float(gh[0] & 0xffff0000u),
                          __uint_as_float(gh[1] << 16), __uint_as_float(gh[1] & 0xffff0000u)};
                u = f32x4{__uint_as_float(uh[0] << 16), __uint_as_float(uh[0] & 0xffff0000u),
                          __uint_as_float(uh[1] << 16), __uint_as_float(uh[1] & 0xffff0000u)};
            } else {
                g = *(const f32x4 *)((const float *)p.G + gi);
                u = *(const f32x4 *)((const float *)p.U + gi);
            }
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                float b;
                dg[e] = silu_grad(v[e], g[e], u[e], b);
                du[e] = b;
            }
            if (p.out_bf16) {
                *(u32x2 *)((uint16_t *)p.C + idx) = u32x2{pack_bf16x2(dg[0], dg[1]), pack_bf16x2(dg[2], dg[3])};
                *(u32x2 *)((uint16_t *)p.C + idx + p.N) = u32x2{pack_bf16x2(du[0], du[1]), pack_bf16x2(du[2], du[3])};
            } else {
                *(f32x4 *)((float *)p.C + idx) = dg;
                *(f32x4 *)((float *)p.C + idx + p.N) = du;
            }
            return;
        }
        if (p.row_scale) v *= p.row_scale[row];
        if (p.beta != 0.f) {
            f32x4 old;
            if (p.out_bf16) {
                const u32x2 o = *(const u32x2 *)((const uint16_t *)p.C + idx);
                old = f32x4{__uint_as_float(o[0] << 16), __uint_as_float(o[0] & 0xffff0000u),
                            __uint_as_float(o[1] << 16), __uint_as_float(o[1] & 0xffff0000u)};
            } else {
                old = *(const f32x4 *)((const float *)p.C + idx);
            }
            v += p.beta * old;
        }
        if (p.has_bias) {
#pragma unroll
            for (int e = 0; e < 4; ++e) v[e] += p.bias[col + e];
        }
        if (p.rope_table && col < p.rope_cols) {
            // col % 4 == 0 and heads have an even width, so both pairs (0,1), (2,3) lie in this vector.
            const float2 *tr = p.rope_table + (row % p.rope_seq) * p.rope_half;
#pragma unroll
            for (int e = 0; e < 4; e += 2) {
                if (col + e >= p.rope_cols) break;
                const float2 cs = tr[((col + e) % (2 * p.rope_half)) / 2];
                const float x0 = v[e], x1 = v[e + 1];
                v[e] = x0 * cs.x - x1 * cs.y;
                v[e + 1] = x0 * cs.y + x1 * cs.x;
            }
        }
        if (p.causal != CAUSAL_NONE) {
#pragma unroll
            for (int e = 0; e < 4; ++e)
                if (col + e > row + p.causal_offset) v[e] = -INFINITY;
        }
        if (p.out_bf16) {
            u32x2 o;
            o[0] = pack_bf16x2(v[0], v[1]);
            o[1] = pack_bf16x2(v[2], v[3]);
            *(u32x2 *)((uint16_t *)p.C + idx) = o;
        } else {
            *(f32x4 *)((float *)p.C + idx) = v;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e)
        if (col + e < p.N) finish_store(p, p.C, idx + e, v[e], row, col + e);
}

// SwiGLU epilogue for 4 consecutive columns: gate = alpha*g (+ gate bias), up = alpha*u (+ up bias
// at bias[N + col]); stores gate and up when asked for, and silu(gate) * up.
template <bool EDGE>
__device__ __forceinline__ void finish_swiglu4(const GemmArgs &p, f32x4 g, f32x4 u, int64_t row, int64_t col,
                                               int64_t coff) {
    if (EDGE && (row >= p.M || col >= p.N)) return;
    g *= p.alpha;
    u *= p.alpha;
    const bool full = !EDGE || col + 4 <= p.N;
    if (p.has_bias) {
#pragma unroll
        for (int e = 0; e < 4; ++e)
            if (full || col + e < p.N) {
                g[e] += p.bias[col + e];
                u[e] += p.bias[p.N + col + e];
            }
    }
    f32x4 h;
#pragma unroll
    for (int e = 0; e < 4; ++e) h[e] = silu(g[e]) * u[e];
    const int64_t idx = coff + row * p.ldc + col;
    if (full && p.c_vec_ok) {
        if (p.out_bf16) {
            auto st = [&](void *dst, f32x4 v) {
                *(u32x2 *)((uint16_t *)dst + idx) = u32x2{pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3])};
            };
            if (p.G) st(p.G, g);
            if (p.U) st(p.U, u);
            st(p.C, h);
        } else {
            if (p.G) *(f32x4 *)((float *)p.G + idx) = g;
            if (p.U) *(f32x4 *)((float *)p.U + idx) = u;
            *(f32x4 *)((float *)p.C + idx) = h;
        }
        return;
    }
#pragma unroll
    for (int e = 0; e < 4; ++e) {
        if (col + e >= p.N) break;
        if (p.G) store_out(p.G, idx + e, g[e], p.out_bf16);
        if (p.U) store_out(p.U, idx + e, u[e], p.out_bf16);
        store_out(p.C, idx + e, h[e], p.out_bf16);
    }
}

}  // namespace
}  // namespace it
