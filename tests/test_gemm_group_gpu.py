"""it_gemm_group (no reference counterpart: the reference's CommandBatch, src/command_batch.rs:166-181,
issues each GEMM separately) on the GPU: the medium step's four weight gradients of one layer
(dW = dY^T . X, K = 8192 tokens: [5632,1024], [3072,1024], [1024,2816], [1024,1024]) run as one
grouped launch of 256 x 256 direct-to-LDS tiles with K unsplit; groups the library does not fuse
(FP32, mixed layouts) run as the separate GEMMs would, bit for bit."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import profiler, synth
from tests.numerics import BF16_FROB_TOL, FP32_TOL, frob_rel, normwise_rel

pytestmark = pytest.mark.gpu

T = 8192
DW = [(5632, 1024), (3072, 1024), (1024, 2816), (1024, 1024)]  # (M, N) of dW = dY^T . X


def _keys(it, fn):
    ctx = it.Context.global_()
    profiler.reset(ctx)
    profiler.enable(ctx)
    fn()
    keys = list(profiler.stats(ctx))
    profiler.enable(ctx, False)
    return keys


def test_group_weight_gradients_exact(it):
    """Small integers: every grouped product equals a float64 product bit for bit on sampled rows
    (exact in any FP32 summation order), the group is one launch, and a second run repeats it."""
    ops = []
    for i, (m, n) in enumerate(DW):
        dy = synth.small_ints(300 + i, (T, m), -2, 2)
        x = synth.small_ints(310 + i, (T, n), -2, 2)
        ops.append((dy, x, it.Tensor.from_f32_as_bf16(dy, dy.shape), it.Tensor.from_f32_as_bf16(x, x.shape),
                    it.Tensor.zeros([m, n])))
    calls = [(a, b, out, True, False) for _, _, a, b, out in ops]
    keys = _keys(it, lambda: it.gemm_group(calls))
    print(f"[group exact] {keys}", flush=True)
    assert len(keys) == 1 and "_dtl_group" in keys[0], keys
    first = [out.numpy() for *_, out in ops]
    rng = np.random.default_rng(3)
    for (dy, x, *_), got, (m, n) in zip(ops, first, DW):
        rows = rng.choice(m, 48, replace=False)
        exact = dy[:, rows].T.astype(np.float64) @ x.astype(np.float64)
        assert np.array_equal(got[rows], exact.astype(np.float32)), (m, n)
    it.gemm_group(calls)
    for (*_, out), f in zip(ops, first):
        assert np.array_equal(out.numpy(), f)


def test_group_matches_separate_and_oracle(it, oracle):
    """Gaussian operands: each grouped FP32 product within the FP32 contract of the oracle on the
    same BF16 operands (sampled rows) and of the separate it_gemm call (which splits K), and within
    the BF16 contract of the unrounded product; the grouped BF16 output is the RNE rounding of the
    grouped FP32 output bit for bit (one accumulation, rounded once)."""
    ops = []
    for i, (m, n) in enumerate(DW):
        dy, x = synth.normal(320 + i, (T, m)), synth.normal(330 + i, (T, n))
        ops.append((dy, x, it.Tensor.from_f32_as_bf16(dy, dy.shape), it.Tensor.from_f32_as_bf16(x, x.shape)))
    got = {}
    for prec in (it.Precision.FP32, it.Precision.BF16):
        outs = [it.Tensor.empty([m, n], prec) for m, n in DW]
        keys = _keys(it, lambda: it.gemm_group([(a, b, o, True, False) for (_, _, a, b), o in zip(ops, outs)]))
        assert len(keys) == 1 and "_dtl_group" in keys[0], keys
        got[prec] = outs
    rng = np.random.default_rng(4)
    for (dy, x, a, b), o32, o16, (m, n) in zip(ops, got[it.Precision.FP32], got[it.Precision.BF16], DW):
        g = o32.numpy()
        sep = it.gemm(a, b, trans_a=True).numpy()
        rows = rng.choice(m, 32, replace=False)
        a_rows = np.ascontiguousarray(dy[:, rows].T)
        ref16 = oracle.gemm_bf16(oracle.f32_to_bf16(a_rows), oracle.f32_to_bf16(x), False, False)
        assert normwise_rel(g[rows], ref16) <= FP32_TOL, (m, n)
        assert normwise_rel(g, sep) <= FP32_TOL, (m, n)
        assert frob_rel(g[rows], oracle.gemm_f32(a_rows, x)) <= BF16_FROB_TOL, (m, n)
        assert np.array_equal(o16.as_bf16_slice().reshape(m, n), oracle.f32_to_bf16(g)), (m, n)


TINY_DW = [(688 * 2, 256), (256, 688), (768, 256), (256, 256)]  # TINY's weight gradients, K = 4096 tokens


def test_group_f32_weight_gradients(it, oracle):
    """FP32: the TINY step's four weight gradients of a layer ([1376,256], [256,688], [768,256],
    [256,256], K = 4096) as one grouped launch of 64 x 64 tiles and one grouped split-K sum: exact
    on small integers (sampled rows against float64), repeatable, and on Gaussian data within the
    FP32 contract of the oracle and of the separate it_gemm calls."""
    k = 4096
    ints, gauss = [], []
    for i, (m, n) in enumerate(TINY_DW):
        dy, x = synth.small_ints(400 + i, (k, m), -2, 2), synth.small_ints(410 + i, (k, n), -2, 2)
        ints.append((dy, x, it.Tensor.from_f32_slice(dy, dy.shape), it.Tensor.from_f32_slice(x, x.shape),
                     it.Tensor.zeros([m, n])))
        gy, gx = synth.normal(420 + i, (k, m)), synth.normal(430 + i, (k, n))
        gauss.append((gy, gx, it.Tensor.from_f32_slice(gy, gy.shape), it.Tensor.from_f32_slice(gx, gx.shape),
                      it.Tensor.zeros([m, n])))
    calls = [(a, b, o, True, False) for _, _, a, b, o in ints]
    keys = _keys(it, lambda: it.gemm_group(calls))
    print(f"[group f32] {keys}", flush=True)
    assert len(keys) == 1 and "f32_TN_64x64_group" in keys[0], keys
    first = [o.numpy() for *_, o in ints]
    rng = np.random.default_rng(6)
    for (dy, x, *_), got in zip(ints, first):
        rows = rng.choice(got.shape[0], 48, replace=False)
        exact = dy[:, rows].T.astype(np.float64) @ x.astype(np.float64)
        assert np.array_equal(got[rows], exact.astype(np.float32)), got.shape
    it.gemm_group(calls)
    for (*_, o), f in zip(ints, first):
        assert np.array_equal(o.numpy(), f)
    it.gemm_group([(a, b, o, True, False) for _, _, a, b, o in gauss])
    for gy, gx, a, b, o in gauss:
        got = o.numpy()
        assert normwise_rel(got, it.gemm(a, b, trans_a=True).numpy()) <= FP32_TOL
        rows = rng.choice(got.shape[0], 32, replace=False)
        ref = oracle.gemm_f32(np.ascontiguousarray(gy[:, rows].T), gx)
        assert normwise_rel(got[rows], ref) <= FP32_TOL


def test_group_fallbacks_equal_separate_calls(it):
    """Groups the library does not fuse run as the separate GEMMs, bit for bit: BF16 GEMMs whose
    tiles exceed one round of CUs, and BF16 GEMMs of two layouts."""
    a16 = it.Tensor.from_f32_as_bf16(synth.normal(350, (4096, 1024)), [4096, 1024])
    w16 = it.Tensor.from_f32_as_bf16(synth.normal(351, (4096, 1024)), [4096, 1024])
    o1, o2 = it.Tensor.zeros([4096, 4096]), it.Tensor.zeros([4096, 4096])
    keys = _keys(it, lambda: it.gemm_group([(a16, w16, o1, False, True), (w16, a16, o2, False, True)]))
    assert keys and not any("_group" in k for k in keys), keys  # one key: both launches have one shape
    assert np.array_equal(o1.numpy(), it.gemm(a16, w16, trans_b=True).numpy())
    assert np.array_equal(o2.numpy(), it.gemm(w16, a16, trans_b=True).numpy())
    b16 = it.Tensor.from_f32_as_bf16(synth.normal(352, (1024, 1024)), [1024, 1024])
    o3, o4 = it.Tensor.zeros([4096, 1024]), it.Tensor.zeros([4096, 1024])
    it.gemm_group([(a16, b16, o3, False, True), (a16, b16, o4, False, False)])
    assert np.array_equal(o3.numpy(), it.gemm(a16, b16, trans_b=True).numpy())
    assert np.array_equal(o4.numpy(), it.gemm(a16, b16).numpy())


def test_group_f32_many_small_gemms_long_k(it):
    """Eight FP32 TN GEMMs with few output tiles and K = 16384 (the group's split count is capped so
    its per-XCD schedule fits the kernel arguments): one grouped launch, exact on small integers
    (every element against float64), repeatable."""
    k = 16384
    shapes = [(64, 128), (128, 64), (64, 64), (192, 64), (64, 256), (128, 128), (64, 64), (256, 64)]
    ops = []
    for i, (m, n) in enumerate(shapes):
        a, b = synth.small_ints(500 + i, (k, m), -2, 2), synth.small_ints(520 + i, (k, n), -2, 2)
        ops.append((a, b, it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape),
                    it.Tensor.zeros([m, n])))
    calls = [(ta, tb, o, True, False) for _, _, ta, tb, o in ops]
    keys = _keys(it, lambda: it.gemm_group(calls))
    print(f"[group f32 long k] {keys}", flush=True)
    assert len(keys) == 1 and "f32_TN_64x64_group" in keys[0], keys
    first = [o.numpy() for *_, o in ops]
    for (a, b, *_), got in zip(ops, first):
        exact = a.T.astype(np.float64) @ b.astype(np.float64)
        assert np.array_equal(got, exact.astype(np.float32)), got.shape
    it.gemm_group(calls)
    for (*_, o), f in zip(ops, first):
        assert np.array_equal(o.numpy(), f)


def test_group_f32_ragged(it, oracle):
    """FP32 TN GEMMs with ragged edges (M and N not multiples of the 64 x 64 tile, K not a multiple
    of the 32-wide k-tile): one grouped launch with bounds-checked loads; exact on small integers
    (every element against float64), and on Gaussian data within the FP32 contract of the oracle."""
    k = 4000
    shapes = [(100, 68), (130, 200), (250, 60), (70, 36)]
    ints, gauss = [], []
    for i, (m, n) in enumerate(shapes):
        a, b = synth.small_ints(600 + i, (k, m), -2, 2), synth.small_ints(610 + i, (k, n), -2, 2)
        ints.append((a, b, it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape),
                     it.Tensor.zeros([m, n])))
        ga, gb = synth.normal(620 + i, (k, m)), synth.normal(630 + i, (k, n))
        gauss.append((ga, gb, it.Tensor.from_f32_slice(ga, ga.shape), it.Tensor.from_f32_slice(gb, gb.shape),
                      it.Tensor.zeros([m, n])))
    calls = [(ta, tb, o, True, False) for _, _, ta, tb, o in ints]
    keys = _keys(it, lambda: it.gemm_group(calls))
    print(f"[group f32 ragged] {keys}", flush=True)
    assert len(keys) == 1 and "f32_TN_64x64_group" in keys[0], keys
    for a, b, *_, o in ints:
        exact = a.T.astype(np.float64) @ b.astype(np.float64)
        assert np.array_equal(o.numpy(), exact.astype(np.float32)), o.shape()
    it.gemm_group([(ta, tb, o, True, False) for _, _, ta, tb, o in gauss])
    for ga, gb, *_, o in gauss:
        ref = oracle.gemm_f32(np.ascontiguousarray(ga.T), gb)
        assert normwise_rel(o.numpy(), ref) <= FP32_TOL, o.shape()


def test_group_f32_graph_replays(it):
    """The FP32 group (split K summed by each tile's last block through the arrival counters),
    captured and replayed three times with eager groups of other operands on the same counters
    between the replays: every replay equals the eager result bit for bit, so each launch leaves
    the counters at zero."""
    import ctypes as C
    from irontensor_amd import _lib
    k = 4096
    ops = []
    for i, (m, n) in enumerate(TINY_DW):
        a, b = synth.small_ints(700 + i, (k, m), -2, 2), synth.small_ints(710 + i, (k, n), -2, 2)
        ops.append((it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape), it.Tensor.zeros([m, n])))
    calls = [(a, b, o, True, False) for a, b, o in ops]
    it.gemm_group(calls)  # eager first: sizes the scratch and allocates the counters
    ref = [o.numpy() for *_, o in ops]
    other = []
    for i, (m, n) in enumerate(TINY_DW):
        a, b = synth.small_ints(720 + i, (k, m), -2, 2), synth.small_ints(730 + i, (k, n), -2, 2)
        other.append((it.Tensor.from_f32_slice(a, a.shape), it.Tensor.from_f32_slice(b, b.shape), it.Tensor.zeros([m, n])))
    other_calls = [(a, b, o, True, False) for a, b, o in other]
    ctx = it.Context.global_()
    ctx.sync()
    assert ctx.lib.it_capture_begin(ctx.handle) == 0
    it.gemm_group(calls)
    graph = C.c_void_p()
    assert ctx.lib.it_capture_end(ctx.handle, C.byref(graph)) == 0, _lib.last_error()
    try:
        for rep in range(3):
            for *_, o in ops:
                zero = np.zeros(o.shape(), np.float32)
                ctx.lib.it_memcpy_h2d(ctx.handle, C.c_void_p(o.ptr), zero.ctypes.data_as(C.c_void_p), zero.nbytes)
            keys = _keys(it, lambda: it.gemm_group(other_calls))  # eager group on the same counters
            assert len(keys) == 1 and "_group" in keys[0], keys
            assert ctx.lib.it_graph_launch(ctx.handle, graph) == 0
            ctx.sync()
            for (*_, o), r in zip(ops, ref):
                assert np.array_equal(o.numpy(), r), rep
    finally:
        ctx.lib.it_graph_destroy(graph)
