"""it_flash_attention_backward_noalloc (the entry point that allocates nothing) against the existing
it_flash_attention_backward, through the C ABI: the two share their kernels and both are
deterministic, so results must be bit-identical. Two calls in a row per dtype, the second smaller
(the static workspace keeps the first call's rows; nothing may leak into the second), a capture of
the call into a HIP graph replayed several times with eager work between the replays, and the
argument checks that refuse what the static workspace cannot hold."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from irontensor_amd import _lib, synth

pytestmark = pytest.mark.gpu

D = 64


def _log(msg):
    print(msg, flush=True)


def _inputs(it, prec, b, h, s, seed):
    P = it.Precision.BF16 if prec == "bf16" else it.Precision.FP32
    q, k, v, do = (synth.normal_tensor(seed + i, (b, h, s, D), precision=P) for i in range(4))
    o, lse = it.flash_attention_forward_bhsd(q, k, v, causal=True, scale=0.125)
    return q, k, v, do, o, lse


def _noalloc(it, prec, q, k, v, do, o, lse, dq, dk, dv):
    b, h, s, _ = q.shape()
    ctx = it.Context.global_()
    lay = _lib.AttnLayout(1, s * D, 0, D)
    dtype = _lib.IT_BF16 if prec == "bf16" else _lib.IT_F32
    vp = lambda t: C.c_void_p(t.ptr) if t is not None else None  # noqa: E731
    return ctx.lib.it_flash_attention_backward_noalloc(
        ctx.handle, dtype, b * h, s, D, C.c_float(0.125), 1, C.byref(lay), None, None,
        vp(do), vp(q), vp(k), vp(v), vp(o), vp(lse), vp(dq), vp(dk), vp(dv))


@pytest.mark.parametrize("prec", ["bf16", "f32"])
def test_noalloc_matches_existing_entry(it, prec):
    for (b, h, s) in ((8, 16, 512), (3, 2, 200)):
        _log(f"[noalloc] {prec} b={b} h={h} s={s}")
        q, k, v, do, o, lse = _inputs(it, prec, b, h, s, 700 + s)
        ref = it.flash_attention_backward(do, q, k, v, causal=True, scale=0.125, o=o, lse=lse)
        got = [it.Tensor.empty([b, h, s, D]) for _ in range(3)]
        assert _noalloc(it, prec, q, k, v, do, o, lse, *got) == 0, _lib.last_error()
        for name, g, r in zip("QKV", got, ref):
            assert np.array_equal(g.numpy(), r.numpy()), (prec, b, h, s, "d" + name)


@pytest.mark.parametrize("prec", ["bf16", "f32"])
def test_noalloc_under_graph_capture(it, prec):
    """Captured without any eager call first (nothing to size, nothing allocated), replayed three
    times; between the replays an eager no-alloc call of another size writes other rows into the
    same static array. Every replay equals the existing entry's result."""
    b, h, s = 4, 8, 384
    q, k, v, do, o, lse = _inputs(it, prec, b, h, s, 760)
    ref = [t.numpy() for t in it.flash_attention_backward(do, q, k, v, causal=True, scale=0.125, o=o, lse=lse)]
    got = [it.Tensor.empty([b, h, s, D]) for _ in range(3)]
    ctx = it.Context.global_()
    ctx.sync()
    _log(f"[noalloc capture] {prec} b={b} h={h} s={s}")
    assert ctx.lib.it_capture_begin(ctx.handle) == 0
    st = _noalloc(it, prec, q, k, v, do, o, lse, *got)
    graph = C.c_void_p()
    assert ctx.lib.it_capture_end(ctx.handle, C.byref(graph)) == 0, _lib.last_error()
    assert st == 0, _lib.last_error()
    try:
        other = _inputs(it, prec, 2, 2, 130, 770)
        other_ref = [t.numpy() for t in it.flash_attention_backward(
            other[3], *other[:3], causal=True, scale=0.125, o=other[4], lse=other[5])]
        other_got = [it.Tensor.empty([2, 2, 130, D]) for _ in range(3)]
        for rep in range(3):
            for t in got:
                t_zero = np.zeros(t.numel(), np.float32)
                ctx.lib.it_memcpy_h2d(ctx.handle, C.c_void_p(t.ptr), t_zero.ctypes.data_as(C.c_void_p), t_zero.nbytes)
            # an eager no-alloc call of another size between replays, on the same static array
            assert _noalloc(it, prec, *other[:3], other[3], other[4], other[5], *other_got) == 0, _lib.last_error()
            assert ctx.lib.it_graph_launch(ctx.handle, graph) == 0
            ctx.sync()
            for name, g, r in zip("QKV", got, ref):
                assert np.array_equal(g.numpy(), r), (rep, "d" + name)
            for name, g, r in zip("QKV", other_got, other_ref):
                assert np.array_equal(g.numpy(), r), (rep, "other d" + name)
    finally:
        ctx.lib.it_graph_destroy(graph)


def test_noalloc_argument_checks(it):
    """Refusals happen on the host before any device work: sizes beyond the static workspace
    (bh * seq > 1048576 rows), and a missing O or lse."""
    small = _inputs(it, "bf16", 1, 1, 64, 780)
    q, k, v, do, o, lse = small
    outs = [it.Tensor.empty([1, 1, 64, D]) for _ in range(3)]
    ctx = it.Context.global_()
    lay = _lib.AttnLayout(1, 0, 0, D)  # a batch stride of 0 keeps every head on the same small buffers
    vp = lambda t: C.c_void_p(t.ptr)  # noqa: E731

    def call(bh, seq, o_, lse_):
        return ctx.lib.it_flash_attention_backward_noalloc(
            ctx.handle, _lib.IT_BF16, bh, seq, D, C.c_float(0.125), 1, C.byref(lay), None, None, vp(do), vp(q),
            vp(k), vp(v), o_, lse_, vp(outs[0]), vp(outs[1]), vp(outs[2]))

    st = call(1025, 1024, vp(o), vp(lse))
    assert st == _lib.IT_ERR_DIMS and "static workspace" in _lib.last_error()
    assert call(1, 64, None, None) == _lib.IT_ERR_NULL
    assert "O and lse are required" in _lib.last_error()
    ctx.sync()
