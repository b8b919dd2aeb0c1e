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
