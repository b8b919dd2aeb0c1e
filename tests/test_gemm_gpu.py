"""GPU parity of the MFMA GEMMs against the CPU oracle, through the C ABI (Python mirror).

FP32: normwise relative error <= 1e-5 against the oracle's sequential f32 loop on the same inputs,
and bit-exact on small-integer inputs (exact arithmetic in any summation order).
BF16: bit-exact on small-integer inputs; relative Frobenius error <= 1e-2 against the f32 oracle on
the unrounded f32 inputs for Gaussian data.
"""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import BF16_FROB_TOL, FP32_TOL, bf16_out_excess, frob_rel, normwise_rel, op

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


# ------------------------------------------------------------------ reference known answers

def test_kat_matmul_2x2(it):
    # src/ops/gemm.rs:291-306
    a = it.Tensor.from_f32_slice([1.0, 2.0, 3.0, 4.0], [2, 2])
    b = it.Tensor.from_f32_slice([5.0, 6.0, 7.0, 8.0], [2, 2])
    c = it.matmul(a, b)
    assert c.shape() == [2, 2]
    assert c.as_f32_slice().tolist() == [19.0, 22.0, 43.0, 50.0]


def test_kat_matmul_larger(it, oracle):
    # src/ops/gemm.rs:308-351 (tolerance 1e-3 absolute there)
    m, k, n = 64, 32, 48
    i, j = np.meshgrid(np.arange(m), np.arange(k), indexing="ij")
    a = (i + j).astype(np.float32) * np.float32(0.01)
    i, j = np.meshgrid(np.arange(k), np.arange(n), indexing="ij")
    b = (i * j).astype(np.float32) * np.float32(0.01)
    c = it.matmul(it.Tensor.from_f32_slice(a, [m, k]), it.Tensor.from_f32_slice(b, [k, n]))
    ref = oracle.gemm_f32(a, b)
    got = c.as_f32_slice().reshape(m, n)
    assert np.max(np.abs(got - ref)) < 1e-3
    assert normwise_rel(got, ref) <= FP32_TOL


def test_kat_matmul_batched(it, oracle):
    # src/ops/gemm.rs:353-386 and src/ops/mps_gemm.rs:612-635
    for (bt, m, k, n) in ((2, 3, 4, 2), (2, 3, 4, 5)):
        a = np.arange(bt * m * k, dtype=np.float32) * np.float32(0.1)
        b = np.arange(bt * k * n, dtype=np.float32) * np.float32(0.1)
        c = it.matmul(it.Tensor.from_f32_slice(a, [bt, m, k]), it.Tensor.from_f32_slice(b, [bt, k, n]))
        assert c.shape() == [bt, m, n]
        ref = oracle.gemm_f32(a.reshape(bt, m, k), b.reshape(bt, k, n))
        assert np.max(np.abs(c.as_f32_slice().reshape(bt, m, n) - ref)) < 1e-3


def test_kat_mps_matches_reference(it):
    # src/ops/mps_gemm.rs:637-668 -- integer data: exact
    m, k, n = 16, 8, 12
    a = ((np.arange(m * k) % 7) - 3).astype(np.float32)
    b = ((np.arange(k * n) % 5) - 2).astype(np.float32)
    c = it.matmul_mps(it.Tensor.from_f32_slice(a, [m, k]), it.Tensor.from_f32_slice(b, [k, n]))
    exact = a.reshape(m, k).astype(np.int64) @ b.reshape(k, n).astype(np.int64)
    assert np.array_equal(c.as_f32_slice().reshape(m, n), exact.astype(np.float32))


def test_kat_matmul_backward(it, oracle):
    # src/ops/backward/gemm.rs:457-586 (2D, batched, 4D)
    for shape_a, shape_b in (([3, 4], [4, 2]), ([2, 3, 4], [2, 4, 2]), ([2, 3, 4, 5], [2, 3, 5, 6])):
        a = (np.arange(np.prod(shape_a), dtype=np.float32) * np.float32(0.01)) % np.float32(1.0)
        b = (np.arange(np.prod(shape_b), dtype=np.float32) * np.float32(0.01)) % np.float32(1.0)
        gshape = shape_a[:-1] + [shape_b[-1]]
        gc = np.ones(int(np.prod(gshape)), np.float32)
        ga, gb = it.matmul_backward(it.Tensor.from_f32_slice(gc, gshape), it.Tensor.from_f32_slice(a, shape_a),
                                    it.Tensor.from_f32_slice(b, shape_b))
        assert ga.shape() == shape_a and gb.shape() == shape_b
        bt = int(np.prod(shape_a[:-2])) if len(shape_a) > 2 else 0
        a3 = a.reshape(([bt] if bt else []) + shape_a[-2:])
        b3 = b.reshape(([bt] if bt else []) + shape_b[-2:])
        g3 = gc.reshape(([bt] if bt else []) + gshape[-2:])
        ref_a = oracle.gemm_f32(g3, b3, trans_b=True)
        ref_b = oracle.gemm_f32(a3, g3, trans_a=True)
        assert np.max(np.abs(ga.as_f32_slice() - ref_a.ravel())) < 1e-4
        assert np.max(np.abs(gb.as_f32_slice() - ref_b.ravel())) < 1e-4


def test_kat_matmul_bf16(it):
    # src/ops/bf16_ops/mod.rs:34-49
    a = it.Tensor.from_f32_as_bf16([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [2, 3])
    b = it.Tensor.from_f32_as_bf16([1.0, 2.0, 3.0, 4.0, 5.0, 6.0], [3, 2])
    c = it.matmul_bf16(a, b)
    assert c.shape() == [2, 2] and c.precision() == it.Precision.BF16
    assert it.bf16_to_f32(c.as_bf16_slice()).tolist() == [22.0, 28.0, 49.0, 64.0]


def test_kat_linear_with_bias(it):
    # src/nn/linear.rs:224-238
    layer = it.Linear.from_weight(it.Tensor.from_f32_slice([1.0, 0.0, 0.0, 1.0], [2, 2]),
                                  it.Tensor.from_f32_slice([1.0, 2.0], [2]))
    out = layer.forward(it.Tensor.from_f32_slice([1.0, 2.0], [1, 2]))
    assert out.as_f32_slice().tolist() == [2.0, 4.0]


# ------------------------------------------------------------------ FP32 parity sweep

SHAPES = [(1, 1, 1), (2, 3, 4), (16, 16, 16), (17, 33, 65), (64, 64, 64), (127, 129, 131),
          (1, 300, 257), (300, 1, 77), (256, 688, 256), (96, 80, 2048)]


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", SHAPES)
def test_f32_parity_layouts(it, oracle, ta, tb, m, n, k):
    _log(f"[f32 parity] ta={ta} tb={tb} m={m} n={n} k={k}")
    a = synth.normal(1000 + m + n, (k, m) if ta else (m, k))
    b = synth.normal(2000 + k, (n, k) if tb else (k, n), std=0.02)
    c = it.gemm(it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape),
                trans_a=bool(ta), trans_b=bool(tb))
    ref = oracle.gemm_f32(a, b, bool(ta), bool(tb))
    assert normwise_rel(c.numpy(), ref) <= FP32_TOL
    # exact arithmetic: small integers give the same bits in any order
    ai = synth.small_ints(3000 + m, a.shape, -3, 3)
    bi = synth.small_ints(4000 + n, b.shape, -3, 3)
    ci = it.gemm(it.Tensor.from_f32_slice(ai, ai.shape), it.Tensor.from_f32_slice(bi, bi.shape),
                 trans_a=bool(ta), trans_b=bool(tb))
    exact = op(ai, ta).astype(np.int64) @ op(bi, tb).astype(np.int64)
    assert np.array_equal(ci.numpy(), exact.astype(np.float32))


def test_config1_qkv_projection(it, oracle):
    """X [4096,256] ~N(0,1), W [768,256] ~N(0,0.02), Y = X.W^T (FP32)."""
    x = synth.normal(1, (4096, 256))
    w = synth.normal(2, (768, 256), std=0.02)
    y = it.matmul_mps_nt(it.Tensor.from_f32_slice(x, x.shape), it.Tensor.from_f32_slice(w, w.shape))
    ref = oracle.gemm_f32(x, w, trans_b=True)
    got = y.numpy()
    err = normwise_rel(got, ref)
    bound = 1e-5 * (np.abs(x).astype(np.float64) @ np.abs(w).astype(np.float64).T)
    _log(f"[config1] normwise rel err {err:.3e}; per-element bound violations "
         f"{int(np.sum(np.abs(got - ref) > bound))}")
    assert err <= FP32_TOL
    assert np.all(np.abs(got - ref) <= bound)


@pytest.mark.parametrize("m,n,k", [(256, 256, 4096), (688, 256, 4096), (256, 16384 // 16, 4096)])
def test_f32_split_k_weight_gradients(it, oracle, m, n, k):
    """dW = dY^T.X (TN) with a long reduction: exercises split-K and its ordered reduction."""
    _log(f"[split-K] m={m} n={n} k={k}")
    dy = synth.normal(5 + m, (k, m))
    x = synth.normal(6 + n, (k, n))
    dw = it.matmul_tn(it.Tensor.from_f32_slice(dy, dy.shape), it.Tensor.from_f32_slice(x, x.shape))
    ref = oracle.gemm_f32(dy, x, trans_a=True)
    assert normwise_rel(dw.numpy(), ref) <= FP32_TOL
    again = it.matmul_tn(it.Tensor.from_f32_slice(dy, dy.shape), it.Tensor.from_f32_slice(x, x.shape))
    assert np.array_equal(dw.numpy(), again.numpy())  # deterministic reduction


def test_f32_alpha_beta_and_broadcast_batch(it, oracle):
    a = synth.normal(7, (3, 40, 24))
    b = synth.normal(8, (24, 56))          # broadcast over the batch
    c0 = synth.normal(9, (3, 40, 56))
    out = it.Tensor.from_f32_slice(c0, c0.shape)
    it.gemm(it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape),
            alpha=0.5, beta=2.0, out=out)
    ref = 0.5 * np.stack([oracle.gemm_f32(a[i], b) for i in range(3)]).astype(np.float64) + 2.0 * c0
    assert normwise_rel(out.numpy(), ref) <= FP32_TOL


def test_f32_bias_epilogue(it, oracle):
    x = synth.normal(10, (2, 33, 96))
    w = synth.normal(11, (80, 96), std=0.02)
    bias = synth.normal(12, (80,))
    y = it.linear(it.Tensor.from_f32_slice(x, x.shape), it.Tensor.from_f32_slice(w, w.shape),
                  it.Tensor.from_f32_slice(bias, bias.shape))
    assert y.shape() == [2, 33, 80]
    ref = oracle.add_bias(oracle.gemm_f32(x.reshape(66, 96), w, trans_b=True), bias)
    assert normwise_rel(y.numpy().reshape(66, 80), ref) <= FP32_TOL


@pytest.mark.parametrize("dtype", ["f32", "bf16"])
def test_causal_epilogue(it, oracle, dtype):
    s, d = 200, 64
    q = synth.normal(13, (s, d))
    k = synth.normal(14, (s, d))
    mk = (lambda x: it.Tensor.from_f32_slice(x, x.shape)) if dtype == "f32" else \
        (lambda x: it.Tensor.from_f32_as_bf16(x, x.shape))
    out = it.gemm(mk(q), mk(k), trans_b=True, alpha=0.125, causal=True).numpy()
    upper = np.triu(np.ones((s, s), bool), 1)
    assert np.all(np.isneginf(out[upper]))
    if dtype == "f32":
        ref = oracle.gemm_f32(q, k, trans_b=True) * np.float32(0.125)
    else:
        ref = oracle.gemm_bf16(oracle.f32_to_bf16(q), oracle.f32_to_bf16(k), trans_b=True) * np.float32(0.125)
    assert normwise_rel(out[~upper], ref[~upper]) <= FP32_TOL


@pytest.mark.parametrize("rows,h,f", [(64, 32, 48), (333, 256, 688)])
def test_f32_swiglu_dual_epilogue(it, oracle, rows, h, f):
    x = synth.normal(15, (rows, h))
    wg = synth.normal(16, (f, h), std=0.05)
    wu = synth.normal(17, (f, h), std=0.05)
    hh, g, u = it.swiglu_up(it.Tensor.from_f32_slice(x, x.shape), it.Tensor.from_f32_slice(wg, wg.shape),
                            it.Tensor.from_f32_slice(wu, wu.shape))
    g_ref = oracle.gemm_f32(x, wg, trans_b=True)
    u_ref = oracle.gemm_f32(x, wu, trans_b=True)
    assert normwise_rel(g.numpy(), g_ref) <= FP32_TOL
    assert normwise_rel(u.numpy(), u_ref) <= FP32_TOL
    assert normwise_rel(hh.numpy(), oracle.swiglu(g_ref, u_ref)) <= FP32_TOL


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_swiglu_dual_epilogue_with_bias(it, oracle, prec):
    """The MED config's fused bias + SwiGLU: gate = x.Wg^T + bg, up = x.Wu^T + bu, h = silu(gate)*up."""
    rows, h, f = 200, 128, 344
    x = synth.normal(18, (rows, h))
    wg = synth.normal(19, (f, h), std=0.05)
    wu = synth.normal(20, (f, h), std=0.05)
    b = synth.normal(21, (2 * f,), std=0.1)
    mk = it.Tensor.from_f32_slice if prec == "f32" else it.Tensor.from_f32_as_bf16
    hh, g, u = it.swiglu_up(mk(x, x.shape), mk(wg, wg.shape), mk(wu, wu.shape),
                            out_precision=it.Precision.FP32, bias=it.Tensor.from_f32_slice(b, [2 * f]))
    g_ref = oracle.add_bias(oracle.gemm_f32(x, wg, trans_b=True), b[:f])
    u_ref = oracle.add_bias(oracle.gemm_f32(x, wu, trans_b=True), b[f:])
    h_ref = oracle.swiglu(g_ref, u_ref)
    if prec == "f32":
        for got, ref in ((g, g_ref), (u, u_ref), (hh, h_ref)):
            assert normwise_rel(got.numpy(), ref) <= FP32_TOL
    else:
        for got, ref in ((g, g_ref), (u, u_ref), (hh, h_ref)):
            assert frob_rel(got.numpy(), ref) <= BF16_FROB_TOL


@pytest.mark.parametrize("rows,h,f", [(4096, 128, 2048), (4000, 200, 2000)])
def test_bf16_swiglu_large_tile(it, oracle, rows, h, f):
    """The 256x256 kernel's dual form (gate and up halves of one B tile, 256 x 128 outputs), exact
    and ragged, with the bias: small integers keep gate and up exact in FP32, so they must equal the
    oracle bit for bit and h = silu(gate) * up must agree to FP32 rounding."""
    from irontensor_amd import profiler
    x = synth.small_ints(220, (rows, h), -2, 2)
    wg = synth.small_ints(221, (f, h), -2, 2)
    wu = synth.small_ints(222, (f, h), -2, 2)
    b = synth.small_ints(223, (2 * f,), -4, 4)
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    hh, g, u = it.swiglu_up(it.Tensor.from_f32_as_bf16(x, x.shape), it.Tensor.from_f32_as_bf16(wg, wg.shape),
                            it.Tensor.from_f32_as_bf16(wu, wu.shape), out_precision=it.Precision.FP32,
                            bias=it.Tensor.from_f32_slice(b, [2 * f]))
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    print(f"[swiglu 256] {keys}", flush=True)
    assert any("256x128" in key and "swiglu" in key for key in keys), keys
    g_ref = oracle.add_bias(oracle.gemm_f32(x, wg, trans_b=True), b[:f])
    u_ref = oracle.add_bias(oracle.gemm_f32(x, wu, trans_b=True), b[f:])
    assert np.array_equal(g.numpy(), g_ref)
    assert np.array_equal(u.numpy(), u_ref)
    assert normwise_rel(hh.numpy(), oracle.swiglu(g_ref, u_ref)) <= FP32_TOL


# ------------------------------------------------------------------ BF16

@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
@pytest.mark.parametrize("m,n,k", [(16, 16, 32), (33, 65, 129), (128, 256, 320), (1, 11008 // 8, 4096)])
def test_bf16_exact_integers(it, oracle, ta, tb, m, n, k):
    _log(f"[bf16 exact] ta={ta} tb={tb} m={m} n={n} k={k}")
    a = synth.small_ints(50 + m, (k, m) if ta else (m, k), -8, 8)
    b = synth.small_ints(60 + n, (n, k) if tb else (k, n), -8, 8)
    ta_, tb_ = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c = it.gemm(ta_, tb_, trans_a=bool(ta), trans_b=bool(tb))
    exact = (op(a, ta).astype(np.int64) @ op(b, tb).astype(np.int64)).astype(np.float32)
    assert np.array_equal(c.numpy(), exact)
    c16 = it.gemm(ta_, tb_, trans_a=bool(ta), trans_b=bool(tb), out_precision=it.Precision.BF16)
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(a), oracle.f32_to_bf16(b), bool(ta), bool(tb), out_bf16=True)
    assert np.array_equal(c16.as_bf16_slice().reshape(ref16.shape), ref16)


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bf16_gaussian_frobenius(it, oracle, ta, tb):
    m, n, k = 512, 384, 1024
    a = synth.normal(70, (k, m) if ta else (m, k))
    b = synth.normal(71, (n, k) if tb else (k, n))
    c = it.gemm(it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape),
                trans_a=bool(ta), trans_b=bool(tb))
    ref = oracle.gemm_f32(a, b, bool(ta), bool(tb))
    err = frob_rel(c.numpy(), ref)
    _log(f"[bf16 frob] ta={ta} tb={tb}: {err:.3e}")
    assert err <= BF16_FROB_TOL
    # against the oracle on the same BF16 operands the only difference is summation order
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(a), oracle.f32_to_bf16(b), bool(ta), bool(tb))
    assert normwise_rel(c.numpy(), ref16) <= FP32_TOL


@pytest.mark.parametrize("m", [1, 4, 16])
@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bf16_decode_shapes(it, oracle, m, ta, tb):
    """BASELINE config 5b: M in {1,4,16}, K=4096, N=11008."""
    k, n = 4096, 11008
    _log(f"[decode] m={m} ta={ta} tb={tb}")
    a = synth.normal(80 + m, (k, m) if ta else (m, k))
    b = synth.normal(81, (n, k) if tb else (k, n))
    c = it.gemm(it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape),
                trans_a=bool(ta), trans_b=bool(tb))
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(a), oracle.f32_to_bf16(b), bool(ta), bool(tb))
    assert normwise_rel(c.numpy(), ref16) <= FP32_TOL
    assert frob_rel(c.numpy(), oracle.gemm_f32(a, b, bool(ta), bool(tb))) <= BF16_FROB_TOL


@pytest.mark.parametrize("m,k,n,ta", [(2, 1000, 1000, 0), (7, 4160, 512, 1), (13, 64, 8, 0), (16, 333, 2056, 1),
                                      (1, 70, 1032, 1)])
def test_bf16_decode_kn_ragged(it, m, k, n, ta):
    """Decode-sized products with the weight stored [K, N] (the tiled GEMM's bounds-checked and
    split-K paths): ragged M, K and column counts, exact small integers against a float64 product,
    plus alpha, beta and bias in the epilogue."""
    _log(f"[decode kn] m={m} k={k} n={n} ta={ta}")
    a = synth.small_ints(210 + m, (k, m) if ta else (m, k), -8, 8)
    b = synth.small_ints(211, (k, n), -8, 8)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c = it.gemm(A, B, trans_a=bool(ta), out_precision=it.Precision.FP32)
    exact = op(a, ta).astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    bias = synth.small_ints(212, (n,), -4, 4)
    c0 = synth.small_ints(213, (m, n), -4, 4)
    out = it.Tensor.from_f32_slice(c0, [m, n])
    it.gemm(A, B, trans_a=bool(ta), alpha=2.0, beta=1.0, out=out, bias=it.Tensor.from_f32_slice(bias, [n]))
    assert np.array_equal(out.numpy(), (2.0 * exact + c0 + bias).astype(np.float32))


@pytest.mark.parametrize("m,k,n", [(1, 4096, 11008), (16, 4096, 11008), (3, 72, 1000), (16, 4104, 77),
                                   (7, 8, 33), (13, 520, 2050), (9, 40, 17), (16, 136, 24)])
def test_bf16_decode_nt_kernel(it, m, k, n):
    """The decode kernel for a weight stored [N, K] (the Linear layout: each load instruction reads 8
    rows x 128 contiguous bytes and DPP moves rearrange each pair of loads into the MFMA operand
    layout): the BASELINE shapes, K not a multiple of 64 or 32, a wave's k range shorter than one
    64-wide block, row and column counts that are not multiples of 8 or 16. Exact small integers
    against a float64 product, BF16 output against the RNE rounding of the exact result, the
    epilogue (alpha, beta, bias), and the plan key names the kernel."""
    from irontensor_amd import profiler
    _log(f"[decode nt kernel] m={m} k={k} n={n}")
    a = synth.small_ints(300 + m, (m, k), -3, 3)
    b = synth.small_ints(301, (n, k), -3, 3)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    c = it.gemm(A, B, trans_b=True, out_precision=it.Precision.FP32)
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    assert any(key.startswith("gemv_bf16_NT") for key in keys), keys
    exact = a.astype(np.float64) @ b.astype(np.float64).T
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    c16 = it.gemm(A, B, trans_b=True, out_precision=it.Precision.BF16)
    assert np.array_equal(c16.as_bf16_slice().reshape(m, n), synth_bf16(exact))
    bias = synth.small_ints(302, (n,), -4, 4)
    c0 = synth.small_ints(303, (m, n), -4, 4)
    out = it.Tensor.from_f32_slice(c0, [m, n])
    it.gemm(A, B, trans_b=True, alpha=2.0, beta=1.0, out=out, bias=it.Tensor.from_f32_slice(bias, [n]))
    assert np.array_equal(out.numpy(), (2.0 * exact + c0 + bias).astype(np.float32))


def test_bf16_decode_nt_batched_and_broadcast(it):
    """The [N, K]-weight decode kernel on a batched product (3 items, each its own weight) and with
    one weight broadcast over the batch."""
    from irontensor_amd import profiler
    bt, m, k, n = 3, 5, 264, 40
    a = synth.small_ints(310, (bt, m, k), -3, 3)
    b = synth.small_ints(311, (bt, n, k), -3, 3)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    c = it.gemm(A, B, trans_b=True)
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    _log(f"[decode nt batched] {keys}")
    assert any(key.startswith("gemv_bf16_NT") for key in keys), keys
    exact = np.matmul(a.astype(np.float64), np.swapaxes(b, 1, 2).astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    b0 = b[0]
    c2 = it.gemm(A, it.Tensor.from_f32_as_bf16(b0, b0.shape), trans_b=True)
    assert np.array_equal(c2.numpy(), np.matmul(a.astype(np.float64), b0.T.astype(np.float64)).astype(np.float32))


@pytest.mark.parametrize("m,k,n,ta", [(1, 4096, 11008, 0), (4, 4096, 11008, 1), (16, 4096, 11008, 0),
                                      (16, 4096, 11008, 1), (5, 1024, 1032, 1), (16, 256, 136, 0), (3, 32, 8, 0)])
def test_bf16_decode_kn_kernel(it, m, k, n, ta):
    """The decode kernel for a weight stored [K, N] (in-register 8 x 8 transposes feeding the MFMA,
    k split over waves and blocks): the BASELINE decode shapes in both layouts, a last column strip
    of 8 columns, one split and a single k chunk. Exact small integers against a float64 product,
    BF16 output against the RNE rounding of the exact result, and the plan key names the kernel."""
    from irontensor_amd import profiler
    _log(f"[decode kn kernel] m={m} k={k} n={n} ta={ta}")
    a = synth.small_ints(260 + m, (k, m) if ta else (m, k), -3, 3)
    b = synth.small_ints(261, (k, n), -3, 3)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    c = it.gemm(A, B, trans_a=bool(ta), out_precision=it.Precision.FP32)
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    _log(f"[decode kn kernel] {keys}")
    assert any(key.startswith("gemv_bf16_TN" if ta else "gemv_bf16_NN") for key in keys), keys
    exact = op(a, ta).astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    c16 = it.gemm(A, B, trans_a=bool(ta), out_precision=it.Precision.BF16)
    assert np.array_equal(c16.as_bf16_slice().reshape(m, n), synth_bf16(exact))


@pytest.mark.parametrize("ta", [0, 1])
def test_bf16_decode_kn_batched_and_broadcast(it, ta):
    """The [K, N]-weight decode kernel on batched products (3 items, each its own weight, split K:
    the arrival counters are per strip and item) and with one weight broadcast over the batch."""
    from irontensor_amd import profiler
    bt, m, k, n = 3, 5, 2048, 264
    a = synth.small_ints(270 + ta, (bt, k, m) if ta else (bt, m, k), -3, 3)
    b = synth.small_ints(272, (bt, k, n), -3, 3)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    c = it.gemm(A, B, trans_a=bool(ta))
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    _log(f"[decode kn batched] ta={ta} {keys}")
    assert any(key.startswith("gemv_bf16_TN" if ta else "gemv_bf16_NN") and not key.endswith(" s1") for key in keys), keys
    exact = np.matmul(op(a, ta).astype(np.float64), b.astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    b0 = b[0]
    c2 = it.gemm(A, it.Tensor.from_f32_as_bf16(b0, b0.shape), trans_a=bool(ta))
    assert np.array_equal(c2.numpy(), np.matmul(op(a, ta).astype(np.float64), b0.astype(np.float64)).astype(np.float32))


def test_bf16_decode_kn_epilogue_after_split_sum(it):
    """alpha, beta and a bias applied by the strip's last block after it adds the split partial sums
    (NN, M = 4: eight k splits)."""
    m, k, n = 4, 4096, 1032
    a = synth.small_ints(280, (m, k), -3, 3)
    b = synth.small_ints(281, (k, n), -3, 3)
    bias = synth.small_ints(282, (n,), -4, 4)
    c0 = synth.small_ints(283, (m, n), -4, 4)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    out = it.Tensor.from_f32_slice(c0, [m, n])
    it.gemm(A, B, alpha=2.0, beta=1.0, out=out, bias=it.Tensor.from_f32_slice(bias, [n]))
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(out.numpy(), (2.0 * exact + c0 + bias).astype(np.float32))


def test_bf16_decode_kn_graph_replays(it):
    """A captured [K, N]-weight decode GEMM (split K, so the captured kernel uses the arrival
    counters) replayed three times with eager decode GEMMs on other shapes between the replays:
    every replay equals the eager result, so each launch leaves the counters at zero."""
    import ctypes as C
    from irontensor_amd import _lib
    m, k, n = 4, 4096, 2056
    a = synth.small_ints(290, (m, k), -3, 3)
    b = synth.small_ints(291, (k, n), -3, 3)
    A, B = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    ref = it.gemm(A, B).numpy()  # eager first: sizes the scratch and allocates the counters
    out = it.Tensor.empty([m, n])
    xo = it.Tensor.from_f32_as_bf16(synth.small_ints(292, (16, k), -3, 3), [16, k])
    ctx = it.Context.global_()
    ctx.sync()
    assert ctx.lib.it_capture_begin(ctx.handle) == 0
    it.gemm(A, B, out=out)
    graph = C.c_void_p()
    assert ctx.lib.it_capture_end(ctx.handle, C.byref(graph)) == 0, _lib.last_error()
    try:
        for rep in range(3):
            zero = np.zeros(m * n, np.float32)
            ctx.lib.it_memcpy_h2d(ctx.handle, C.c_void_p(out.ptr), zero.ctypes.data_as(C.c_void_p), zero.nbytes)
            other = it.gemm(xo, B)  # eager work on the same counters between the replays
            assert ctx.lib.it_graph_launch(ctx.handle, graph) == 0
            ctx.sync()
            assert np.array_equal(out.numpy(), ref), rep
            assert other.shape() == [16, n]
    finally:
        ctx.lib.it_graph_destroy(graph)
    assert np.array_equal(ref, (a.astype(np.float64) @ b.astype(np.float64)).astype(np.float32))


def synth_bf16(x):
    """RNE rounding of float64 values (exactly representable in FP32 here) to BF16 bits."""
    from oracle import f32_to_bf16
    return f32_to_bf16(np.asarray(x, dtype=np.float32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
def test_bf16_square_1024_against_oracle(it, oracle, ta, tb):
    """BASELINE config 5a at n = 1024 in the NN, NT and TN layouts, whole output against the oracle:
    normwise 1e-5 against its FP32 sums of the same BF16 operands, relative Frobenius 1e-2 against
    its f32 loop on the unrounded N(0,1) inputs."""
    n = 1024
    _log(f"[square 1024] ta={ta} tb={tb}")
    a = synth.normal(95, (n, n))
    b = synth.normal(96, (n, n))
    a16, b16 = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
    c = it.gemm(it.Tensor.from_bf16_slice(a16, a.shape), it.Tensor.from_bf16_slice(b16, b.shape),
                trans_a=bool(ta), trans_b=bool(tb)).numpy()
    assert normwise_rel(c, oracle.gemm_bf16(a16, b16, bool(ta), bool(tb))) <= FP32_TOL
    assert frob_rel(c, oracle.gemm_f32(a, b, bool(ta), bool(tb))) <= BF16_FROB_TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0)])
@pytest.mark.parametrize("n", [2048, 4096, 8192, 16384])
def test_bf16_square_full_size(it, n, ta, tb):
    """BASELINE config 5a at full size, NN / NT / TN (the oracle's loop would take minutes to hours):
    * Freivalds: (op(A).op(B)).x == op(A).(op(B).x) in float64 for a random x, on the BF16 operands,
      error relative to |op(A)|.(|op(B)|.|x|) below 1e-5;
    * 64+ sampled full output rows against a float64 product of the same BF16 operands (normwise
      1e-5) and of the unrounded seeded N(0,1) inputs regenerated on the host (Frobenius 1e-2).
    The operands are drawn on the device (synth.normal_tensor, the stream of synth.normal)."""
    from tests.stepcheck import sample_rows
    _log(f"[square full] n={n} ta={ta} tb={tb}")
    seed_a, seed_b = 90 + n, 91 + n
    A = synth.normal_tensor(seed_a, (n, n), precision=it.Precision.BF16)
    B = synth.normal_tensor(seed_b, (n, n), precision=it.Precision.BF16)
    c = it.gemm(A, B, trans_a=bool(ta), trans_b=bool(tb)).numpy()
    a64 = it.bf16_to_f32(A.as_bf16_slice()).reshape(n, n).astype(np.float64)
    b64 = it.bf16_to_f32(B.as_bf16_slice()).reshape(n, n).astype(np.float64)
    opa = a64.T if ta else a64
    opb = b64.T if tb else b64
    x = synth.normal(92, (n,)).astype(np.float64)
    lhs = c.astype(np.float64) @ x
    rhs = opa @ (opb @ x)
    scale = np.abs(opa) @ (np.abs(opb) @ np.abs(x))
    fv = float(np.max(np.abs(lhs - rhs) / scale))
    rows = sample_rows(n, 64, seed=n + 3 * ta + tb)
    ref_same = opa[rows] @ opb
    e_same = normwise_rel(c[rows], ref_same)
    _log(f"[square full] n={n} ta={ta} tb={tb}: freivalds {fv:.2e}, rows same-operand {e_same:.2e}")
    assert fv < 1e-5
    assert e_same <= FP32_TOL
    if n <= 8192:
        # unrounded inputs (host generation of n^2 normals; 16384^2 would take most of a minute):
        # element (i, j) of the stored matrix is normal number i * n + j of its seed
        ia = (np.arange(n)[:, None] * n + rows[None, :]) if ta else (rows[:, None] * n + np.arange(n)[None, :])
        a_rows = synth.normal_at(seed_a, ia).astype(np.float64)
        a_rows = a_rows.T if ta else a_rows
        b32 = synth.normal(seed_b, (n, n)).astype(np.float64)
        e_frob = frob_rel(c[rows], a_rows @ (b32.T if tb else b32))
        _log(f"[square full] n={n}: frob vs unrounded {e_frob:.2e}")
        assert e_frob <= BF16_FROB_TOL


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_large_tile_ragged_batched(it, ta, tb):
    """Ragged batched shapes big enough for the 256x256 kernel's bounds-checked path: exact small
    integers, checked against a float64 product (exact for these magnitudes)."""
    bt, m, n, k = 24, 740, 730, 136
    a = synth.small_ints(200, (bt, k, m) if ta else (bt, m, k), -8, 8)
    b = synth.small_ints(201, (bt, n, k) if tb else (bt, k, n), -8, 8)
    c = it.gemm(it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape),
                trans_a=bool(ta), trans_b=bool(tb))
    exact = np.matmul(op(a, ta).astype(np.float64), op(b, tb).astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(5632, 1024, 8192), (1000, 2800, 8010)])
def test_bf16_large_tile_split_k(it, m, n, k):
    """Long-K weight-gradient shapes take a 256x256 kernel with split-K: whole tiles (the medium
    step's up/gate dW, on the direct-to-LDS kernel) and ragged (the register-staged kernel); the
    profiler key shows the plan. Small integers: exact in BF16 and in every FP32 summation order,
    checked against a float64 product."""
    a = synth.small_ints(210, (k, m), -2, 2)
    b = synth.small_ints(211, (k, n), -2, 2)
    ta, tb = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    from irontensor_amd import profiler
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    c = it.gemm(ta, tb, trans_a=True)
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    print(f"[split-K 256] {keys}", flush=True)
    assert any("256x256" in key and not key.endswith(" s1") for key in keys), keys
    exact = a.T.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    again = it.gemm(ta, tb, trans_a=True)
    assert np.array_equal(c.numpy(), again.numpy())  # ordered reduction: deterministic


def _plan_keys(it, fn):
    from irontensor_amd import profiler
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    out = fn()
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    return out, keys


@pytest.mark.parametrize("ta,tb,m,n,k", [(1, 0, 1024, 2816, 8192), (0, 0, 8192, 2816, 1024), (0, 1, 8192, 1024, 1024),
                                         (1, 1, 3072, 1024, 8192), (1, 0, 5632, 1024, 8192)])
def test_bf16_uneven_tile_counts_exact(it, ta, tb, m, n, k):
    """The medium step's shapes whose 256x256 tiles do not fill the CUs evenly (44, 352, 128, 48
    and 88 tiles) in every layout, on the direct-to-LDS kernel (whole tiles, split-K or a partial
    round): small integers are exact in every FP32 summation order, so the result must equal a
    float64 product bit for bit, and a second run must repeat it."""
    a = synth.small_ints(230 + m, (k, m) if ta else (m, k), -2, 2)
    b = synth.small_ints(231 + n, (n, k) if tb else (k, n), -2, 2)
    at, bt = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c, keys = _plan_keys(it, lambda: it.gemm(at, bt, trans_a=bool(ta), trans_b=bool(tb)))
    _log(f"[uneven tiles exact] ta={ta} tb={tb} {m}x{n}x{k}: {keys}")
    assert any("_dtl" in key for key in keys), keys
    exact = np.matmul(op(a, ta).astype(np.float64), op(b, tb).astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    again = it.gemm(at, bt, trans_a=bool(ta), trans_b=bool(tb))
    assert np.array_equal(c.numpy(), again.numpy())


@pytest.mark.parametrize("ta,tb,m,n,k", [(0, 0, 4096, 1152, 1024), (0, 1, 4096, 1152, 2048), (1, 0, 1536, 1024, 8192),
                                         (1, 1, 4096, 1152, 256), (0, 0, 8192, 1024, 1024)])
def test_bf16_dtl_256x128_exact(it, ta, tb, m, n, k):
    """The 256 x 128 direct-to-LDS tile (each wave 128 x 64; B staged as 128 rows) in every
    layout: N an odd multiple of 128 rules the 256 x 256 tile out, the medium step's N = 1024
    data gradient takes it to fill the CUs, and a 1536 x 1024 weight gradient with split-K.
    Small integers are exact in any FP32 summation order: the result equals a float64 product
    bit for bit, and a second run repeats it."""
    a = synth.small_ints(250 + m, (k, m) if ta else (m, k), -2, 2)
    b = synth.small_ints(251 + n, (n, k) if tb else (k, n), -2, 2)
    at, bt = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c, keys = _plan_keys(it, lambda: it.gemm(at, bt, trans_a=bool(ta), trans_b=bool(tb)))
    _log(f"[256x128 exact] ta={ta} tb={tb} {m}x{n}x{k}: {keys}")
    assert any("256x128_dtl" in key for key in keys), keys
    exact = np.matmul(op(a, ta).astype(np.float64), op(b, tb).astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    again = it.gemm(at, bt, trans_a=bool(ta), trans_b=bool(tb))
    assert np.array_equal(c.numpy(), again.numpy())


def test_bf16_dtl_256x128_epilogues(it, oracle):
    """The 256 x 128 tile's epilogues: alpha/beta into a BF16 output (exact on small integers),
    a bias with FP32 output, a bias with BF16 output (the rounding of the FP32 result), and
    Gaussian operands within the FP32 contract of the oracle on the same BF16 values."""
    m, n, k = 4096, 1152, 256
    a = synth.small_ints(260, (m, k), -4, 4)
    b = synth.small_ints(261, (n, k), -4, 4)
    c0 = synth.small_ints(262, (m, n), -4, 4)
    at, bt = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    out = it.Tensor.from_f32_as_bf16(c0, c0.shape)
    _, keys = _plan_keys(it, lambda: it.gemm(at, bt, trans_b=True, alpha=0.5, beta=2.0, out=out))
    _log(f"[256x128 epilogues] {keys}")
    assert any("256x128_dtl" in key for key in keys), keys
    exact = 0.5 * (a.astype(np.float64) @ b.astype(np.float64).T) + 2.0 * c0
    assert np.array_equal(out.as_bf16_slice().reshape(m, n), oracle.f32_to_bf16(exact.astype(np.float32)))
    bias = synth.normal(263, (n,))
    tbias = it.Tensor.from_f32_slice(bias, bias.shape)
    y = it.gemm(at, bt, trans_b=True, bias=tbias)
    ref = (a.astype(np.float64) @ b.astype(np.float64).T) + bias
    assert normwise_rel(y.numpy(), ref) <= FP32_TOL
    y16 = it.gemm(at, bt, trans_b=True, bias=tbias, out_precision=it.Precision.BF16)
    assert bf16_out_excess(y16.numpy(), ref) <= FP32_TOL
    ga, gb = synth.normal(264, (m, 2 * k)), synth.normal(265, (2 * k, n))
    g, keys = _plan_keys(it, lambda: it.gemm(it.Tensor.from_f32_as_bf16(ga, ga.shape),
                                             it.Tensor.from_f32_as_bf16(gb, gb.shape)))
    assert any("256x128_dtl" in key for key in keys), keys
    rows = np.random.default_rng(8).choice(m, 256, replace=False)
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(np.ascontiguousarray(ga[rows])), oracle.f32_to_bf16(gb), False, False)
    assert normwise_rel(g.numpy()[rows], ref16) <= FP32_TOL


def test_bf16_long_k_gaussian(it, oracle):
    """The medium step's down.dW shape (K = 8192 tokens, 44 tiles, split-K) on Gaussian data: 64
    sampled output rows within the FP32 contract of the oracle on the same BF16 operands and
    within the BF16 contract of the unrounded product; the BF16 output equals the rounding of the
    FP32 result to the FP32 contract."""
    m, n, k = 1024, 2816, 8192
    a = synth.normal(240, (k, m))
    b = synth.normal(241, (k, n))
    at, bt = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c, keys = _plan_keys(it, lambda: it.gemm(at, bt, trans_a=True))
    _log(f"[long-K gaussian] {keys}")
    rows = np.random.default_rng(7).choice(m, 64, replace=False)
    a_rows = np.ascontiguousarray(a[:, rows].T)
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(a_rows), oracle.f32_to_bf16(b), False, False)
    got = c.numpy()[rows]
    assert normwise_rel(got, ref16) <= FP32_TOL
    assert frob_rel(got, oracle.gemm_f32(a_rows, b)) <= BF16_FROB_TOL
    c16 = it.gemm(at, bt, trans_a=True, out_precision=it.Precision.BF16)
    assert bf16_out_excess(c16.numpy()[rows], ref16) <= FP32_TOL


def test_bf16_swiglu_medium_shape(it, oracle):
    """The SwiGLU dual form at the medium step's gate|up projection shape (704 tiles of 256 x 128,
    the direct-to-LDS kernel's paired epilogue): gate and up exact on small integers, h =
    silu(gate) * up to FP32 rounding."""
    rows, h, f = 8192, 1024, 2816
    x = synth.small_ints(250, (rows, h), -2, 2)
    wg = synth.small_ints(251, (f, h), -2, 2)
    wu = synth.small_ints(252, (f, h), -2, 2)
    (hh, g, u), keys = _plan_keys(it, lambda: it.swiglu_up(
        it.Tensor.from_f32_as_bf16(x, x.shape), it.Tensor.from_f32_as_bf16(wg, wg.shape),
        it.Tensor.from_f32_as_bf16(wu, wu.shape), out_precision=it.Precision.FP32))
    _log(f"[swiglu medium] {keys}")
    assert any("_dtl_swiglu" in key for key in keys), keys
    xd = x.astype(np.float64)
    g_ref = (xd @ wg.astype(np.float64).T).astype(np.float32)
    u_ref = (xd @ wu.astype(np.float64).T).astype(np.float32)
    assert np.array_equal(g.numpy(), g_ref)
    assert np.array_equal(u.numpy(), u_ref)
    rows_chk = np.arange(0, rows, 61)
    assert normwise_rel(hh.numpy()[rows_chk], oracle.swiglu(g_ref[rows_chk], u_ref[rows_chk])) <= FP32_TOL


def test_bf16_large_tile_epilogues(it, oracle):
    """alpha/beta with BF16 output and a bias on a shape that takes the 256x256 kernel."""
    m, n, k = 4096, 3072, 192
    a = synth.small_ints(210, (m, k), -4, 4)
    b = synth.small_ints(211, (n, k), -4, 4)
    c0 = synth.small_ints(212, (m, n), -4, 4)
    out = it.Tensor.from_f32_as_bf16(c0, c0.shape)
    it.gemm(it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape),
            trans_b=True, alpha=0.5, beta=2.0, out=out)
    exact = 0.5 * (a.astype(np.float64) @ b.astype(np.float64).T) + 2.0 * c0
    ref16 = oracle.f32_to_bf16(exact.astype(np.float32))
    assert np.array_equal(out.as_bf16_slice().reshape(m, n), ref16)
    bias = synth.normal(213, (n,))
    y = it.gemm(it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape),
                trans_b=True, bias=it.Tensor.from_f32_slice(bias, bias.shape))
    ref = (a.astype(np.float64) @ b.astype(np.float64).T) + bias
    assert normwise_rel(y.numpy(), ref) <= FP32_TOL


@pytest.mark.parametrize("layout", ["NT", "NN", "TN", "TT"])
@pytest.mark.parametrize("m,n,k", [(1536, 1536, 1536), (2048, 2048, 2048), (1920, 1280, 1344)])
def test_bf16_128_tile_exact(it, m, n, k, layout):
    """BF16 products at shapes the planner runs on the 128 x 128 direct-to-LDS tile (four LDS
    stages; 1344 = 21 k-tiles, an odd count), in every layout (a transposed operand is read through
    transposing LDS reads): exact on small integers against a float64 product (every partial sum is
    an integer below 2^15, exact in float64 and in FP32)."""
    from irontensor_amd import profiler
    ta, tb = layout[0] == "T", layout[1] == "T"
    x = synth.small_ints(800 + m, (k, m) if ta else (m, k), -3, 3)
    w = synth.small_ints(801 + n, (n, k) if tb else (k, n), -3, 3)
    tx, tw = it.Tensor.from_f32_as_bf16(x, x.shape), it.Tensor.from_f32_as_bf16(w, w.shape)
    out = it.Tensor.zeros([m, n])
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    it.gemm(tx, tw, trans_a=ta, trans_b=tb, out=out)
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    print(f"[bf16 128 {layout}] {keys}", flush=True)
    assert "128x128_dtl" in keys[0], keys
    ref = (x.T if ta else x).astype(np.float64) @ (w.T if tb else w).astype(np.float64)
    assert np.array_equal(out.numpy(), ref.astype(np.float32))


@pytest.mark.parametrize("ta,tb", [(0, 0), (0, 1), (1, 0), (1, 1)])
def test_bf16_128_tile_batched_exact(it, ta, tb):
    """Batched BF16 products whose 128 x 128 tiles fill the CUs only across the batch (4 x 64
    tiles of [1024, 1024, 1024]) run on the 128 x 128 direct-to-LDS tile in every layout, the batch
    index on the grid's second axis: exact on small integers against a float64 product (exact at
    these magnitudes), and a B shared by the whole batch (batch stride 0) gives the same result as
    the B repeated."""
    bt, m, n, k = 4, 1024, 1024, 1024
    a = synth.small_ints(870, (bt, k, m) if ta else (bt, m, k), -3, 3)
    b = synth.small_ints(871, (bt, n, k) if tb else (bt, k, n), -3, 3)
    at, bt_ = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c, keys = _plan_keys(it, lambda: it.gemm(at, bt_, trans_a=bool(ta), trans_b=bool(tb)))
    _log(f"[128 batched exact] ta={ta} tb={tb}: {keys}")
    assert any("128x128_dtl" in key for key in keys), keys
    exact = np.matmul(op(a, ta).astype(np.float64), op(b, tb).astype(np.float64))
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    b0 = b[0]
    shared = it.gemm(at, it.Tensor.from_f32_as_bf16(b0, b0.shape), trans_a=bool(ta), trans_b=bool(tb))
    exact0 = np.matmul(op(a, ta).astype(np.float64), op(b0, tb).astype(np.float64))
    assert np.array_equal(shared.numpy(), exact0.astype(np.float32))


@pytest.mark.parametrize("m,n,k", [(1024, 1024, 8192), (512, 1024, 16384), (1024, 896, 4096)])
def test_bf16_128_tile_split_k_exact(it, m, n, k):
    """Long-K weight gradients (A transposed) whose 128 x 128 tiles are too few for the CUs run on
    that tile with split-K (the medium step's 1024 x 1024 weight gradient, and 4-8 splits): exact on
    small integers against a float64 product, and a second run repeats it (ordered reduction)."""
    a = synth.small_ints(860 + m, (k, m), -2, 2)
    b = synth.small_ints(861 + n, (k, n), -2, 2)
    at, bt = it.Tensor.from_f32_as_bf16(a, a.shape), it.Tensor.from_f32_as_bf16(b, b.shape)
    c, keys = _plan_keys(it, lambda: it.gemm(at, bt, trans_a=True))
    _log(f"[128 split-K exact] {m}x{n}x{k}: {keys}")
    assert any("128x128_dtl" in key and not key.endswith(" s1") for key in keys), keys
    exact = a.T.astype(np.float64) @ b.astype(np.float64)
    assert np.array_equal(c.numpy(), exact.astype(np.float32))
    again = it.gemm(at, bt, trans_a=True)
    assert np.array_equal(c.numpy(), again.numpy())


@pytest.mark.parametrize("tb", [False, True])
def test_f32_256_tile_exact(it, tb):
    """FP32 data gradients of the LM-head shape ([4096, 256, 16384], X.W and X.W^T) run on the
    256 x 128 FP32 tile with split K (one block per CU): exact on small integers against a float64
    product (every partial sum is an integer below 2^24), with alpha and a bias in the epilogue
    that follows the split-K reduction."""
    from irontensor_amd import profiler
    m, n, k = 4096, 256, 16384
    x = synth.small_ints(820, (m, k), -3, 3)
    w = synth.small_ints(821, (n, k) if tb else (k, n), -3, 3)
    bias = synth.small_ints(822, (n,), -4, 4)
    tx, tw = it.Tensor.from_f32_slice(x, list(x.shape)), it.Tensor.from_f32_slice(w, list(w.shape))
    out = it.Tensor.zeros([m, n])
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    it.gemm(tx, tw, trans_b=tb, out=out, alpha=2.0, bias=it.Tensor.from_f32_slice(bias, [n]))
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    print(f"[f32 256] tb={tb} {keys}", flush=True)
    assert keys[0].startswith("gemm_f32_N") and "_256x128|" in keys[0] and not keys[0].endswith(" s1"), keys
    ref = x.astype(np.float64) @ (w.T if tb else w).astype(np.float64)  # exact: integers below 2^53
    assert np.array_equal(out.numpy(), (2 * ref + bias).astype(np.float32))


@pytest.mark.parametrize("m,n,k,lay", [(4096, 256, 1376, "NN"), (4096, 256, 688, "NT"), (4096, 256, 256, "NN"),
                                       (4000, 250, 700, "NT"), (4000, 250, 700, "TN"), (1000, 90, 300, "NN")])
def test_f32_64x32_tile_exact(it, m, n, k, lay):
    """FP32 GEMMs the planner runs on the 64 x 32 tile (two blocks per CU where 64 x 64 tiles leave
    one): the TINY step's [4096, 256, K] data gradients and projections, and ragged shapes (masked or
    bounds-checked loads at every edge). Exact on small integers against a float64 product, with
    alpha and a bias in the epilogue; the TINY shapes' plan key names the tile."""
    from irontensor_amd import profiler
    ta, tb = lay[0] == "T", lay[1] == "T"
    a = synth.small_ints(840 + m % 7, (k, m) if ta else (m, k), -3, 3)
    b = synth.small_ints(841 + n % 7, (n, k) if tb else (k, n), -3, 3)
    bias = synth.small_ints(842, (n,), -4, 4)
    A, B = it.Tensor.from_f32_slice(a, list(a.shape)), it.Tensor.from_f32_slice(b, list(b.shape))
    out = it.Tensor.zeros([m, n])
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    it.gemm(A, B, trans_a=ta, trans_b=tb, out=out, alpha=2.0, bias=it.Tensor.from_f32_slice(bias, [n]))
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    print(f"[f32 64x32] {m}x{n}x{k} {lay} {keys}", flush=True)
    if m == 4096:
        assert "_64x32|" in keys[0], keys
    ref = op(a, ta).astype(np.float64) @ (b.T if tb else b).astype(np.float64)
    assert np.array_equal(out.numpy(), (2 * ref + bias).astype(np.float32))
