"""Per-launch timing from the library's profiler (hipEvents around every launch on the context's
stream, keyed by kernel, plan and shape). The reference's Profiler (src/profile/mod.rs:238) times command
buffers; this is its counterpart for this path."""
from __future__ import annotations

import ctypes as C
import json

from .errors import check


def enable(ctx, on: bool = True) -> None:
    check(ctx.lib.it_profiler_enable(ctx.handle, int(on)), "profiler")


def reset(ctx) -> None:
    check(ctx.lib.it_profiler_reset(ctx.handle), "profiler")


def stats(ctx) -> dict:
    """{key: {"calls": n, "total_ms": t, ...}} for everything launched while enabled."""
    need = C.c_size_t(0)
    ctx.lib.it_profiler_report(ctx.handle, None, 0, C.byref(need))
    buf = C.create_string_buffer(need.value + 16)
    check(ctx.lib.it_profiler_report(ctx.handle, buf, need.value + 16, C.byref(need)), "profiler")
    return json.loads(buf.value.decode())


def matmul_by_shape(ctx) -> dict:
    """The reference report's "Matmul by Shape" (Profiler::record_matmul_shape, src/ops/mps_gemm.rs:22-30;
    src/profile/report.rs:198-230): {"[4096,256]x[768,256]^T": {"count": n, "total_ms": t}, ...} over
    every GEMM launched while enabled, whatever kernel and plan ran it."""
    need = C.c_size_t(0)
    ctx.lib.it_profiler_report_shapes(ctx.handle, None, 0, C.byref(need))
    buf = C.create_string_buffer(need.value + 16)
    check(ctx.lib.it_profiler_report_shapes(ctx.handle, buf, need.value + 16, C.byref(need)), "profiler")
    return json.loads(buf.value.decode())
