"""GPU parity of the boundary ops that the reference re-exports beside its GEMMs
(src/ops/mod.rs:21, src/train/helpers.rs:12-83, src/ops/gemm.rs:102, src/ops/bf16_ops/gemm.rs:85-146),
through the C ABI (Python mirror), against the oracle:

* transpose_3d_gpu and causal_mask_3d_gpu: bit-exact (they move or replace values; nothing is
  computed), at ragged shapes and at the TINY / ATTN attention shapes, plus the in-place mask;
* linear_backward and ensure_fp32 with FP32 and BF16 weights: FP32 normwise 1e-5;
* matmul_custom: FP32 normwise 1e-5, errors as panics;
* matmul_bf16_batched with BF16 output: bit-exact on small integers (exact in every order), and on
  Gaussian data within half a BF16 ulp of the oracle's FP32 sum plus the FP32 contract;
* the seeded device fill: the host generator's stream.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import (BF16_FROB_TOL, FP32_TOL, bf16_out_excess, frob_rel, normwise_rel)

pytestmark = pytest.mark.gpu


def _log(msg):
    print(msg, flush=True)


@pytest.mark.parametrize("batch,m,n", [(1, 1, 1), (2, 3, 5), (3, 70, 130), (5, 64, 128), (64, 256, 64),
                                       (128, 1024, 64), (7, 1, 300)])
def test_transpose_3d_gpu(it, oracle, batch, m, n):
    _log(f"[transpose_3d] batch={batch} m={m} n={n}")
    x = synth.normal(300 + m + n, (batch, m, n))
    got = it.transpose_3d_gpu(it.Tensor.from_f32_slice(x, x.shape), batch, m, n)
    assert got.shape() == [batch, n, m]
    assert np.array_equal(got.numpy(), oracle.transpose_3d(x, batch, m, n))


def test_transpose_3d_gpu_errors_and_empty(it):
    t = it.Tensor.from_f32_slice(np.zeros(12, np.float32), [2, 2, 3])
    with pytest.raises(it.Panic, match="Tensor size mismatch"):
        it.transpose_3d_gpu(t, 2, 2, 4)
    e = it.transpose_3d_gpu(it.Tensor.empty([0, 4, 5]), 0, 4, 5)
    assert e.shape() == [0, 5, 4]
    lib, ctx = it.Context.global_().lib, it.Context.global_()
    st = lib.it_transpose_3d(ctx.handle, C.c_void_p(t.ptr), C.c_void_p(t.ptr), 2, 2, 3)
    assert st == 5  # IT_ERR_INVALID: the output may not overlap the input


@pytest.mark.parametrize("batch,seq", [(1, 1), (3, 37), (2, 130), (64, 256), (128, 1024)])
def test_causal_mask_3d_gpu(it, oracle, batch, seq):
    _log(f"[causal_mask_3d] batch={batch} seq={seq}")
    x = synth.normal(310 + seq, (batch, seq, seq))
    ref = oracle.causal_mask_3d(x, batch, seq)
    got = it.causal_mask_3d_gpu(it.Tensor.from_f32_slice(x, x.shape), batch, seq).numpy()
    assert np.array_equal(got.view(np.uint32), ref.view(np.uint32))
    # in place, through the C ABI (the reference always writes a new tensor; in == out is allowed)
    t = it.Tensor.from_f32_slice(x, x.shape)
    ctx = it.Context.global_()
    assert ctx.lib.it_causal_mask_3d(ctx.handle, C.c_void_p(t.ptr), C.c_void_p(t.ptr), batch, seq) == 0
    assert np.array_equal(t.numpy().view(np.uint32), ref.view(np.uint32))


def test_causal_mask_3d_gpu_errors(it):
    with pytest.raises(it.Panic, match="Tensor size mismatch"):
        it.causal_mask_3d_gpu(it.Tensor.from_f32_slice(np.zeros(8, np.float32), [2, 2, 2]), 2, 3)
    assert it.causal_mask_3d_gpu(it.Tensor.empty([0, 3, 3]), 0, 3).shape() == [0, 3, 3]


@pytest.mark.parametrize("wprec", ["f32", "bf16"])
def test_linear_backward_and_ensure_fp32(it, oracle, wprec):
    """src/train/helpers.rs:12-18, 48-76: (dX, dW) = (dY.W, dY^T.X), with a BF16 weight widened to
    FP32 first (ensure_fp32); linear_forward through the same widening."""
    t, fin, fout = 512, 256, 768
    x = synth.normal(320, (t, fin))
    w = synth.normal(321, (fout, fin), std=0.02)
    dy = synth.normal(322, (t, fout))
    tx, tdy = it.Tensor.from_f32_slice(x, x.shape), it.Tensor.from_f32_slice(dy, dy.shape)
    if wprec == "bf16":
        tw = it.Tensor.from_f32_as_bf16(w, w.shape)
        w_eff = oracle.bf16_to_f32(oracle.f32_to_bf16(w))
        widened = it.ensure_fp32(tw)
        assert widened.precision() == it.Precision.FP32
        assert np.array_equal(widened.numpy(), w_eff)  # exact widening, src/precision.rs:33-35
    else:
        tw = it.Tensor.from_f32_slice(w, w.shape)
        w_eff = w
        assert it.ensure_fp32(tw) is tw  # FP32 passes through (the reference's clone shares the buffer)
    y = it.linear_forward(tx, tw)
    assert normwise_rel(y.numpy(), oracle.gemm_f32(x, w_eff, trans_b=True)) <= FP32_TOL
    dx, dw = it.linear_backward(tdy, tx, tw)
    assert dx.precision() == it.Precision.FP32 and dw.precision() == it.Precision.FP32
    assert normwise_rel(dx.numpy(), oracle.gemm_f32(dy, w_eff)) <= FP32_TOL
    assert normwise_rel(dw.numpy(), oracle.gemm_f32(dy, x, trans_a=True)) <= FP32_TOL


@pytest.mark.parametrize("shape_a,shape_b", [([64, 32], [32, 48]), ([3, 33, 65], [3, 65, 17]),
                                             ([300, 700], [700, 260])])
def test_matmul_custom(it, oracle, shape_a, shape_b):
    """src/ops/gemm.rs:102-285: the custom-kernel matmul, 2D and batched, panicking on bad input."""
    a = synth.normal(330 + shape_a[-1], shape_a)
    b = synth.normal(331 + shape_b[-1], shape_b)
    c = it.matmul_custom(it.Tensor.from_f32_slice(a, shape_a), it.Tensor.from_f32_slice(b, shape_b))
    assert normwise_rel(c.numpy(), oracle.gemm_f32(a, b)) <= FP32_TOL
    with pytest.raises(it.Panic):
        it.matmul_custom(it.Tensor.from_f32_slice(a, shape_a), it.Tensor.from_f32_slice(a, shape_a))


@pytest.mark.parametrize("bt,m,k,n", [(2, 3, 4, 2), (4, 33, 65, 17), (6, 128, 256, 192), (3, 300, 520, 260)])
def test_matmul_bf16_batched_bf16_output(it, oracle, bt, m, k, n):
    """src/ops/bf16_ops/gemm.rs:85-146: BF16 [B,M,K].[B,K,N] -> BF16, FP32 accumulation, RNE of the
    sum (src/shaders/bf16_ops.metal:93)."""
    _log(f"[matmul_bf16_batched] bt={bt} m={m} k={k} n={n}")
    ai = synth.small_ints(340 + m, (bt, m, k), -8, 8)
    bi = synth.small_ints(341 + n, (bt, k, n), -8, 8)
    c = it.matmul_bf16_batched(it.Tensor.from_f32_as_bf16(ai, ai.shape), it.Tensor.from_f32_as_bf16(bi, bi.shape))
    assert c.shape() == [bt, m, n] and c.precision() == it.Precision.BF16
    ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(ai), oracle.f32_to_bf16(bi), out_bf16=True)
    assert np.array_equal(c.as_bf16_slice().reshape(ref16.shape), ref16)
    a = synth.normal(342 + m, (bt, m, k))
    b = synth.normal(343 + n, (bt, k, n))
    a16, b16 = oracle.f32_to_bf16(a), oracle.f32_to_bf16(b)
    c = it.matmul_bf16_batched(it.Tensor.from_bf16_slice(a16, a.shape), it.Tensor.from_bf16_slice(b16, b.shape))
    got = c.numpy()
    assert bf16_out_excess(got, oracle.gemm_bf16(a16, b16)) <= FP32_TOL
    assert frob_rel(got, oracle.gemm_f32(a, b)) <= BF16_FROB_TOL
    with pytest.raises(it.Panic):
        it.matmul_bf16_batched(it.Tensor.from_bf16_slice(a16, a.shape), it.Tensor.from_bf16_slice(a16, a.shape))


@pytest.mark.parametrize("prec", ["f32", "bf16"])
def test_fill_normal_is_the_host_stream(it, prec):
    """it_fill_normal writes synth.normal's values: bit for bit, except where the device's float64
    log/sin/cos and the host libm's differ by an ulp that moves the FP32 rounding (then by one
    FP32 ulp); offsets and odd lengths select the same elements."""
    P = it.Precision.FP32 if prec == "f32" else it.Precision.BF16
    n = 1_000_003
    host = synth.normal(350, (n,), std=0.02)
    t = synth.normal_tensor(350, (n,), std=0.02, precision=P)
    got = t.numpy().ravel()
    want = host if prec == "f32" else it.bf16_to_f32(it.f32_to_bf16(host))
    differ = np.flatnonzero(got.view(np.uint32) != want.view(np.uint32))
    _log(f"[fill_normal {prec}] {differ.size} of {n} elements differ")
    assert differ.size <= 4
    ulps = np.abs(got.view(np.int32)[differ].astype(np.int64) - want.view(np.int32)[differ])
    assert np.all(ulps <= (1 if prec == "f32" else 1 << 16))
    # an element range from an odd offset
    ctx = it.Context.global_()
    part = it.Tensor.empty([1001], it.Precision.FP32)
    assert ctx.lib.it_fill_normal(ctx.handle, 0, 350, 12345, 1001, 0.02, C.c_void_p(part.ptr)) == 0
    ref = synth.normal_at(350, np.arange(12345, 12345 + 1001), std=0.02)
    assert np.max(np.abs(part.numpy().view(np.int32).astype(np.int64) - ref.view(np.int32))) <= 1


def test_profiler_matmul_by_shape(it):
    """The library profiler's GEMM launches keyed as the reference's Profiler::record_matmul_shape
    keys them (src/ops/mps_gemm.rs:22-30,421-422): A and B as stored, "^T" on a transposed operand;
    a grouped launch counts once per GEMM."""
    from irontensor_amd import profiler
    ctx = it.Context.global_()
    x = it.Tensor.from_f32_slice(synth.normal(1, (4096, 256)), [4096, 256])
    w = it.Tensor.from_f32_slice(synth.normal(2, (768, 256), std=0.02), [768, 256])
    a = it.Tensor.from_f32_slice(synth.normal(3, (64, 32)), [64, 32])
    b = it.Tensor.from_f32_slice(synth.normal(4, (32, 48)), [32, 48])
    dy = it.Tensor.from_f32_slice(synth.normal(5, (4096, 768)), [4096, 768])
    profiler.reset(ctx)
    profiler.enable(ctx)
    it.matmul_mps_nt(x, w)
    it.matmul_mps_nt(x, w)
    it.matmul(a, b)
    it.matmul_mps_tn(dy, x)
    shapes = profiler.matmul_by_shape(ctx)
    profiler.enable(ctx, False)
    print(f"[profiler shapes] {shapes}", flush=True)
    assert shapes["[4096,256]x[768,256]^T"]["count"] == 2
    assert shapes["[64,32]x[32,48]"]["count"] == 1
    assert shapes["[4096,768]^Tx[4096,256]"]["count"] == 1
    assert all(v["total_ms"] > 0 for v in shapes.values())
