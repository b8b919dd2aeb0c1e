"""The runtime's graph and scratch lifetime on the GPU: a graph captured over library scratch keeps
working after a later, larger eager call has replaced that scratch (the old block is retired until
the last graph is destroyed), replayed asynchronously as the reference's commit_async allows
(src/command_batch.rs:228-272). Runs on a context of its own so the sizes it grows are known."""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

from irontensor_amd import _lib, synth

pytestmark = pytest.mark.gpu

MIB = 1 << 20


def test_graph_survives_scratch_grow(it):
    ctx = it.Context(0)  # a fresh context: its scratch starts empty
    lib = ctx.lib
    try:
        assert lib.it_mem_scratch(ctx.handle) == 0
        b, h, s, d = 2, 4, 256, 64
        q, k, v, do = (it.Tensor.from_f32_slice(synth.normal(900 + i, (b, h, s, d)), [b, h, s, d], ctx)
                       for i in range(4))
        # Eager first: the fused backward that recomputes its forward sizes the attention scratch.
        ref = [t.numpy() for t in it.flash_attention_backward(do, q, k, v, causal=True)]
        first = lib.it_mem_scratch(ctx.handle)
        assert first >= 64 * MIB
        outs = [it.Tensor.empty([b, h, s, d], ctx=ctx) for _ in range(3)]
        lay = _lib.AttnLayout(1, s * d, 0, d)
        vp = lambda t: C.c_void_p(t.ptr)  # noqa: E731
        ctx.sync()
        print("[graph/scratch] capturing the fused backward", flush=True)
        assert lib.it_capture_begin(ctx.handle) == 0
        st = lib.it_flash_attention_backward(ctx.handle, _lib.IT_F32, b * h, s, d, C.c_float(0.125), 1,
                                             C.byref(lay), None, None, vp(do), vp(q), vp(k), vp(v), None, None,
                                             *(vp(t) for t in outs))
        graph = C.c_void_p()
        assert lib.it_capture_end(ctx.handle, C.byref(graph)) == 0, _lib.last_error()
        assert st == 0, _lib.last_error()
        try:
            # A larger eager call on the same scratch: head_dim 32 runs the materialised attention,
            # whose score buffers (2 * 16 * 1024 * 1024 * 4 B = 128 MiB) outgrow the first block.
            big = [it.Tensor.from_f32_slice(synth.normal(910 + i, (4, 4, 1024, 32)), [4, 4, 1024, 32], ctx)
                   for i in range(3)]
            print("[graph/scratch] eager call that grows the scratch", flush=True)
            it.flash_attention(*big, True)
            ctx.sync()
            grown = lib.it_mem_scratch(ctx.handle)
            assert grown >= first + 128 * MIB  # the old block is retired, not freed
            for rep in range(3):
                for t in outs:
                    assert lib.it_zero(ctx.handle, vp(t), t.byte_size()) == 0
                print(f"[graph/scratch] replay {rep}", flush=True)
                assert lib.it_graph_launch(ctx.handle, graph) == 0, _lib.last_error()
                # eager work between replays, on the grown scratch
                it.flash_attention(*big, True)
                ctx.sync()
                for name, t, r in zip("QKV", outs, ref):
                    assert np.array_equal(t.numpy(), r), (rep, "d" + name)
        finally:
            assert lib.it_graph_destroy(graph) == 0
        # With no graph left the retired block is released.
        assert lib.it_mem_scratch(ctx.handle) == grown - first
    finally:
        lib.it_shutdown(ctx.handle)
        ctx.handle = None


def test_graph_replays_only_on_its_context(it):
    """A graph holds its context's buffers and scratch, so another context may not replay it."""
    a, b = it.Context(0), it.Context(0)
    lib = a.lib
    try:
        t = it.Tensor.from_f32_slice(np.ones(1024, dtype=np.float32), [1024], a)
        a.sync()
        assert lib.it_capture_begin(a.handle) == 0
        st = lib.it_zero(a.handle, C.c_void_p(t.ptr), t.byte_size())
        graph = C.c_void_p()
        assert lib.it_capture_end(a.handle, C.byref(graph)) == 0, _lib.last_error()
        assert st == 0, _lib.last_error()
        try:
            assert lib.it_graph_launch(b.handle, graph) == _lib.IT_ERR_INVALID
            assert "another context" in _lib.last_error()
            assert lib.it_graph_launch(a.handle, graph) == 0, _lib.last_error()
            a.sync()
            assert not t.numpy().any()
        finally:
            assert lib.it_graph_destroy(graph) == 0
    finally:
        for c in (a, b):
            lib.it_shutdown(c.handle)
            c.handle = None
