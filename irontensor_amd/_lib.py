"""ctypes binding of libirontensor_hip.so (the C ABI declared in include/irontensor_hip.h).

Loading never falls back to anything: if the library is missing the import of the op layer fails
with a message that says how to build it.
"""
from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

LIB_PATH = Path(os.environ.get("IRONTENSOR_LIB") or Path(__file__).resolve().parent / "libirontensor_hip.so")

IT_OK = 0
IT_ERR_INNER_DIM = 1
IT_ERR_SHAPE = 2
IT_ERR_PRECISION = 3
IT_ERR_DIMS = 4
IT_ERR_INVALID = 5
IT_ERR_NULL = 6
IT_ERR_OOM = 7
IT_ERR_NO_DEVICE = 8
IT_ERR_HIP = 9
IT_ERR_NOT_READY = 10

IT_F32, IT_F16, IT_BF16 = 0, 1, 2
IT_OP_N, IT_OP_T = 0, 1

IT_EPI_BIAS = 0x1
IT_EPI_SWIGLU = 0x2
IT_EPI_CAUSAL = 0x4
IT_EPI_ROPE = 0x8
IT_EPI_SWIGLU_BWD = 0x10
IT_EPI_XENT_A = 0x20

c_void_p = C.c_void_p
c_i64 = C.c_int64
c_int = C.c_int
c_float = C.c_float


class Epilogue(C.Structure):
    _fields_ = [
        ("flags", C.c_uint32),
        ("bias", c_void_p),
        ("B2", c_void_p),
        ("gate_out", c_void_p),
        ("up_out", c_void_p),
        ("causal_offset", c_i64),
        ("rope_base", c_float),
        ("rope_seq", c_i64),
        ("rope_head_dim", c_i64),
        ("rope_cols", c_i64),
        ("rope_offset", c_i64),
        ("xent_stats", c_void_p),
        ("xent_targets", c_void_p),
        ("xent_scale", c_float),
    ]


class GemmCall(C.Structure):
    """One GEMM of it_gemm_group (it_gemm's arguments after the dtypes)."""
    _fields_ = [
        ("transA", C.c_int),
        ("transB", C.c_int),
        ("M", c_i64),
        ("N", c_i64),
        ("K", c_i64),
        ("alpha", c_float),
        ("A", c_void_p),
        ("lda", c_i64),
        ("strideA", c_i64),
        ("B", c_void_p),
        ("ldb", c_i64),
        ("strideB", c_i64),
        ("beta", c_float),
        ("C", c_void_p),
        ("ldc", c_i64),
        ("strideC", c_i64),
        ("batch", c_i64),
        ("epi", C.POINTER(Epilogue)),
    ]


class AttnLayout(C.Structure):
    _fields_ = [
        ("heads", c_i64),
        ("batch_stride", c_i64),
        ("head_stride", c_i64),
        ("row_stride", c_i64),
    ]


# name -> (restype, argtypes)
_SIGNATURES = {
    "it_init": (c_int, [c_int, C.POINTER(c_void_p)]),
    "it_shutdown": (c_int, [c_void_p]),
    "it_last_error": (C.c_char_p, []),
    "it_status_string": (C.c_char_p, [c_int]),
    "it_device_count": (c_int, []),
    "it_device_info": (c_int, [c_void_p, C.c_char_p, C.c_size_t, C.POINTER(c_int), C.POINTER(c_int)]),
    "it_malloc": (c_int, [c_void_p, C.c_size_t, C.POINTER(c_void_p)]),
    "it_free": (c_int, [c_void_p, c_void_p]),
    "it_mem_allocated": (C.c_size_t, [c_void_p]),
    "it_mem_scratch": (C.c_size_t, [c_void_p]),
    "it_empty_cache": (c_int, [c_void_p]),
    "it_memcpy_h2d": (c_int, [c_void_p, c_void_p, c_void_p, C.c_size_t]),
    "it_memcpy_d2h": (c_int, [c_void_p, c_void_p, c_void_p, C.c_size_t]),
    "it_memcpy_d2d": (c_int, [c_void_p, c_void_p, c_void_p, C.c_size_t]),
    "it_zero": (c_int, [c_void_p, c_void_p, C.c_size_t]),
    "it_stream_sync": (c_int, [c_void_p]),
    "it_stream": (c_void_p, [c_void_p]),
    "it_event_create": (c_int, [c_void_p, C.POINTER(c_void_p)]),
    "it_event_record": (c_int, [c_void_p, c_void_p]),
    "it_event_query": (c_int, [c_void_p]),
    "it_event_sync": (c_int, [c_void_p]),
    "it_event_elapsed_ms": (c_int, [c_void_p, c_void_p, C.POINTER(c_float)]),
    "it_event_destroy": (c_int, [c_void_p]),
    "it_gemm": (c_int, [c_void_p, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64, c_float,
                        c_void_p, c_i64, c_i64, c_void_p, c_i64, c_i64, c_float,
                        c_void_p, c_i64, c_i64, c_i64, C.POINTER(Epilogue)]),
    "it_gemm_group": (c_int, [c_void_p, c_int, c_int, c_int, C.POINTER(GemmCall)]),
    "it_gemm_check": (c_int, [c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64,
                              c_void_p, c_i64, c_i64, c_void_p, c_i64, c_i64, c_float,
                              c_void_p, c_i64, c_i64, c_i64, C.POINTER(Epilogue)]),
    "it_f32_to_bf16": (c_int, [c_void_p, c_void_p, c_void_p, c_i64]),
    "it_bf16_to_f32": (c_int, [c_void_p, c_void_p, c_void_p, c_i64]),
    "it_softmax_rows": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_i64, c_i64, c_i64, c_int, c_i64]),
    "it_softmax_backward": (c_int, [c_void_p, c_void_p, c_void_p, c_int, c_void_p, c_int,
                                    c_i64, c_i64, c_i64, c_int]),
    "it_attention_forward": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_float, c_int,
                                     C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                     C.POINTER(AttnLayout),
                                     c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "it_attention_backward": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_float, c_int,
                                      C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                      C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p, c_void_p,
                                      c_void_p, c_void_p, c_void_p]),
    "it_flash_attention_forward": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_i64, c_float, c_int,
                                           C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                           C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p,
                                           c_void_p, c_void_p]),
    "it_flash_attention_backward": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_float, c_int,
                                            C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                            C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p,
                                            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "it_flash_attention_forward_ex": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_float, c_int,
                                              C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                              C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_void_p]),
    "it_flash_attention_backward_ex": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_float, c_int,
                                               C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                               C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p,
                                               c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "it_flash_attention_backward_noalloc": (c_int, [c_void_p, c_int, c_i64, c_i64, c_i64, c_float, c_int,
                                                    C.POINTER(AttnLayout), C.POINTER(AttnLayout),
                                                    C.POINTER(AttnLayout), c_void_p, c_void_p, c_void_p,
                                                    c_void_p, c_void_p, c_void_p, c_void_p, c_void_p,
                                                    c_void_p]),
    "it_rmsnorm_forward": (c_int, [c_void_p, c_int, c_i64, c_i64, c_float, c_void_p, c_void_p, c_void_p,
                                   c_void_p, c_void_p]),
    "it_rmsnorm_backward": (c_int, [c_void_p, c_i64, c_i64, c_float, c_void_p, c_void_p, c_void_p, c_void_p,
                                    c_void_p, c_void_p]),
    "it_rope": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_i64, c_float, c_i64, c_int,
                        c_void_p, c_i64, c_void_p, c_i64, c_i64]),
    "it_embedding_forward": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p]),
    "it_embedding_backward": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p]),
    "it_cross_entropy_fused": (c_int, [c_void_p, c_int, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p,
                                       c_void_p]),
    "it_cross_entropy_stats": (c_int, [c_void_p, c_i64, c_i64, c_void_p, c_void_p, c_void_p, c_void_p, c_void_p]),
    "it_swiglu_backward": (c_int, [c_void_p, c_int, c_int, c_i64, c_i64, c_void_p, c_i64, c_void_p, c_void_p,
                                   c_i64, c_void_p, c_void_p, c_i64]),
    "it_grad_norm_clip": (c_int, [c_void_p, c_int, C.POINTER(c_void_p), C.POINTER(c_i64), c_float, c_void_p]),
    "it_lion_step": (c_int, [c_void_p, c_int, C.POINTER(c_void_p), C.POINTER(c_void_p), C.POINTER(c_void_p),
                             C.POINTER(c_i64), c_float, c_float, c_float, c_float, c_void_p, c_void_p]),
    "it_fused_rmsnorm_linear": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_float, c_void_p, c_void_p, c_void_p,
                                        c_void_p]),
    "it_fused_linear_cross_entropy": (c_int, [c_void_p, c_i64, c_i64, c_i64, c_void_p, c_void_p, c_void_p,
                                              c_void_p, c_void_p, c_void_p, c_void_p, c_i64]),
    "it_transpose_3d": (c_int, [c_void_p, c_void_p, c_void_p, c_i64, c_i64, c_i64]),
    "it_causal_mask_3d": (c_int, [c_void_p, c_void_p, c_void_p, c_i64, c_i64]),
    "it_fill_normal": (c_int, [c_void_p, c_int, C.c_uint64, c_i64, c_i64, C.c_double, c_void_p]),
    "it_side_begin": (c_int, [c_void_p]),
    "it_side_end": (c_int, [c_void_p]),
    "it_side_join": (c_int, [c_void_p]),
    "it_capture_begin": (c_int, [c_void_p]),
    "it_capture_end": (c_int, [c_void_p, C.POINTER(c_void_p)]),
    "it_graph_launch": (c_int, [c_void_p, c_void_p]),
    "it_graph_destroy": (c_int, [c_void_p]),
    "it_profiler_enable": (c_int, [c_void_p, c_int]),
    "it_profiler_reset": (c_int, [c_void_p]),
    "it_profiler_report": (c_int, [c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
    "it_profiler_report_shapes": (c_int, [c_void_p, C.c_char_p, C.c_size_t, C.POINTER(C.c_size_t)]),
}

_lib = None


def load() -> C.CDLL:
    """Loads the in-tree library once and declares every signature."""
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(
            f"{LIB_PATH} is missing: build it with `python -m irontensor_amd.build` "
            "(or __graft_entry__.build()); there is no fallback implementation")
    lib = C.CDLL(str(LIB_PATH))
    for name, (res, args) in _SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _lib = lib
    return lib


def last_error() -> str:
    return load().it_last_error().decode(errors="replace")


def status_name(st: int) -> str:
    return load().it_status_string(st).decode()
