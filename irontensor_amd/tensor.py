"""Device context and Tensor: the runtime under the matmul path, over the C ABI.

Mirrors the reference's MetalContext (src/device.rs:10-71), CommandBatch sync points
(src/command_batch.rs:166-391) and Tensor (src/tensor.rs:11-302) for discrete HBM: a Tensor owns a
refcounted device buffer from the library's caching allocator; host reads (`as_f32_slice`,
`as_bf16_slice`) synchronise the stream and copy out, as the reference's reads of unified memory
happen after a sync.
"""
from __future__ import annotations

import ctypes as C
import enum
from typing import Sequence

import numpy as np

from . import _lib
from .errors import DeviceError, Panic, check


class Precision(enum.IntEnum):
    """src/precision.rs:1-16 (same order as it_dtype)."""

    FP32 = 0
    FP16 = 1
    BF16 = 2

    def byte_size(self) -> int:
        return 4 if self is Precision.FP32 else 2


# ------------------------------------------------------------------ host-side BF16 (precision.rs)

def f32_to_bf16(x) -> np.ndarray:
    """src/precision.rs:24-29, vectorised: bits + (0x7FFF + ((bits >> 16) & 1)) wrapping, >> 16."""
    bits = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    rnd = ((bits >> np.uint32(16)) & np.uint32(1)) + np.uint32(0x7FFF)
    with np.errstate(over="ignore"):
        return ((bits + rnd) >> np.uint32(16)).astype(np.uint16)


def bf16_to_f32(x) -> np.ndarray:
    """src/precision.rs:33-35."""
    return (np.ascontiguousarray(x, dtype=np.uint16).astype(np.uint32) << np.uint32(16)).view(np.float32)


# ------------------------------------------------------------------ context

class Context:
    """One device, one HIP stream (replaces MetalContext::global, src/device.rs:15-29)."""

    _global: "Context | None" = None

    def __init__(self, device: int = 0):
        self.lib = _lib.load()
        handle = C.c_void_p()
        check(self.lib.it_init(device, C.byref(handle)), "it_init")
        self.handle = handle
        self.device = device

    @classmethod
    def global_(cls) -> "Context":
        if cls._global is None:
            cls._global = Context(0)
        return cls._global

    def sync(self) -> None:
        """CommandBatch::sync."""
        check(self.lib.it_stream_sync(self.handle), "sync")

    def memory_allocated(self) -> int:
        """gpu_memory_allocated (src/device.rs:43-71)."""
        return int(self.lib.it_mem_allocated(self.handle))

    def info(self) -> dict:
        name = C.create_string_buffer(256)
        cus, clk = C.c_int(), C.c_int()
        check(self.lib.it_device_info(self.handle, name, 256, C.byref(cus), C.byref(clk)))
        return {"arch": name.value.decode(), "compute_units": cus.value, "clock_khz": clk.value}


def device_count() -> int:
    return int(_lib.load().it_device_count())


class _Buffer:
    """A device allocation shared by a tensor and its views."""

    __slots__ = ("ctx", "ptr", "nbytes", "__weakref__")

    def __init__(self, ctx: Context, nbytes: int):
        self.ctx = ctx
        ptr = C.c_void_p()
        check(ctx.lib.it_malloc(ctx.handle, max(int(nbytes), 1), C.byref(ptr)), "alloc")
        self.ptr = ptr.value
        self.nbytes = int(nbytes)

    def __del__(self):
        try:
            if self.ptr:
                self.ctx.lib.it_free(self.ctx.handle, C.c_void_p(self.ptr))
                self.ptr = None
        except Exception:
            pass


def _numel(shape: Sequence[int]) -> int:
    n = 1
    for d in shape:
        n *= int(d)
    return n


class Tensor:
    """Contiguous row-major device tensor (src/tensor.rs:11-302)."""

    __slots__ = ("_buf", "_shape", "_precision")

    def __init__(self, buf: _Buffer, shape: Sequence[int], precision: Precision):
        self._buf = buf
        self._shape = [int(d) for d in shape]
        self._precision = Precision(precision)

    # ---- constructors
    @staticmethod
    def empty(shape: Sequence[int], precision: Precision = Precision.FP32, ctx: Context | None = None) -> "Tensor":
        """Uninitialised device tensor (outputs that a kernel fully overwrites)."""
        ctx = ctx or Context.global_()
        return Tensor(_Buffer(ctx, _numel(shape) * Precision(precision).byte_size()), shape, precision)

    @staticmethod
    def zeros(shape: Sequence[int], precision: Precision = Precision.FP32, ctx: Context | None = None) -> "Tensor":
        t = Tensor.empty(shape, precision, ctx)
        if t.byte_size():
            check(t._buf.ctx.lib.it_zero(t._buf.ctx.handle, C.c_void_p(t.ptr), t.byte_size()), "zeros")
        return t

    @staticmethod
    def _upload(arr: np.ndarray, shape, precision: Precision, ctx: Context | None) -> "Tensor":
        n = _numel(shape)
        if arr.size != n:
            raise Panic(f"Data length {arr.size} does not match shape {list(shape)} (numel={n})")
        t = Tensor.empty(shape, precision, ctx)
        if n:
            arr = np.ascontiguousarray(arr)
            check(t._buf.ctx.lib.it_memcpy_h2d(t._buf.ctx.handle, C.c_void_p(t.ptr),
                                              arr.ctypes.data_as(C.c_void_p), arr.nbytes), "upload")
        return t

    @staticmethod
    def from_f32_slice(data, shape: Sequence[int], ctx: Context | None = None) -> "Tensor":
        return Tensor._upload(np.asarray(data, dtype=np.float32).ravel(), shape, Precision.FP32, ctx)

    @staticmethod
    def from_bf16_slice(data, shape: Sequence[int], ctx: Context | None = None) -> "Tensor":
        return Tensor._upload(np.asarray(data, dtype=np.uint16).ravel(), shape, Precision.BF16, ctx)

    @staticmethod
    def from_f32_as_bf16(data, shape: Sequence[int], ctx: Context | None = None) -> "Tensor":
        return Tensor.from_bf16_slice(f32_to_bf16(np.asarray(data, dtype=np.float32).ravel()), shape, ctx)

    # ---- metadata
    def shape(self) -> list:
        return list(self._shape)

    def precision(self) -> Precision:
        return self._precision

    def numel(self) -> int:
        return _numel(self._shape)

    def byte_size(self) -> int:
        return self.numel() * self._precision.byte_size()

    def is_bf16(self) -> bool:
        return self._precision is Precision.BF16

    def is_f32(self) -> bool:
        return self._precision is Precision.FP32

    @property
    def ptr(self) -> int:
        return self._buf.ptr

    @property
    def ctx(self) -> Context:
        return self._buf.ctx

    # ---- host access (synchronising copies)
    def _download(self, dtype) -> np.ndarray:
        out = np.empty(self.numel(), dtype=dtype)
        if out.size:
            check(self.ctx.lib.it_memcpy_d2h(self.ctx.handle, out.ctypes.data_as(C.c_void_p),
                                             C.c_void_p(self.ptr), out.nbytes), "download")
        return out

    def as_f32_slice(self) -> np.ndarray:
        if self._precision is not Precision.FP32:
            raise Panic("Tensor precision is not FP32")
        return self._download(np.float32)

    def as_bf16_slice(self) -> np.ndarray:
        if self._precision is not Precision.BF16:
            raise Panic("Tensor precision is not BF16")
        return self._download(np.uint16)

    def numpy(self) -> np.ndarray:
        """Host copy shaped like the tensor (BF16 widened to float32)."""
        if self._precision is Precision.BF16:
            return bf16_to_f32(self.as_bf16_slice()).reshape(self._shape)
        return self.as_f32_slice().reshape(self._shape)

    # ---- views
    def view(self, new_shape: Sequence[int]) -> "Tensor":
        n = _numel(new_shape)
        if n != self.numel():
            raise Panic(f"Cannot view tensor of {self.numel()} elements as shape {list(new_shape)} ({n} elements)")
        return Tensor(self._buf, new_shape, self._precision)

    def reshape(self, new_shape: Sequence[int]) -> None:
        n = _numel(new_shape)
        if n != self.numel():
            raise Panic(f"Cannot reshape tensor of {self.numel()} elements to shape {list(new_shape)} ({n} elements)")
        self._shape = [int(d) for d in new_shape]

    def clone(self) -> "Tensor":
        t = Tensor.empty(self._shape, self._precision, self.ctx)
        if self.byte_size():
            check(self.ctx.lib.it_memcpy_d2d(self.ctx.handle, C.c_void_p(t.ptr), C.c_void_p(self.ptr),
                                             self.byte_size()), "clone")
        return t

    # ---- precision conversion (CPU, as src/tensor.rs:268-292)
    def to_bf16(self) -> "Tensor":
        if self._precision is not Precision.FP32:
            raise Panic("to_bf16() requires FP32 tensor")
        return Tensor.from_bf16_slice(f32_to_bf16(self.as_f32_slice()), self._shape, self.ctx)

    def to_f32(self) -> "Tensor":
        if self._precision is not Precision.BF16:
            raise Panic("to_f32() requires BF16 tensor")
        return Tensor.from_f32_slice(bf16_to_f32(self.as_bf16_slice()), self._shape, self.ctx)

    def __repr__(self) -> str:
        return f"Tensor(shape={self._shape}, precision={self._precision.name}, ptr=0x{self.ptr or 0:x})"


__all__ = ["Context", "Tensor", "Precision", "f32_to_bf16", "bf16_to_f32", "device_count", "DeviceError"]
