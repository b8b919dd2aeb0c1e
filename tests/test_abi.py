"""CPU tests of the C-ABI library: it loads, exports every declared symbol, and rejects bad
arguments with the reference's error kinds before touching a device. No compute calls."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import pytest

from irontensor_amd import _lib
from irontensor_amd.tensor import Precision, Tensor

ROOT = Path(__file__).resolve().parents[1]


def declared_functions():
    names = set()
    for hdr in (ROOT / "include").glob("*.h"):
        text = re.sub(r"/\*.*?\*/", "", hdr.read_text(), flags=re.S)
        names.update(re.findall(r"\b(it_[a-z0-9_]+)\s*\(", text))
    return sorted(names)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing
    # and the ctypes layer declares a signature for each of them
    assert set(names) <= set(_lib._SIGNATURES), set(names) - set(_lib._SIGNATURES)


def test_status_strings():
    lib = _lib.load()
    for st in range(0, 11):
        assert lib.it_status_string(st).decode() not in ("", "unknown status")
    assert lib.it_status_string(99).decode() == "unknown status"


def _check(**kw):
    args = dict(dtype_in=_lib.IT_F32, dtype_out=_lib.IT_F32, ta=0, tb=0, M=4, N=5, K=6,
                A=16, lda=6, sA=0, B=16, ldb=5, sB=0, beta=0.0, Cp=16, ldc=5, sC=0, batch=1, epi=None)
    args.update(kw)
    lib = _lib.load()
    st = lib.it_gemm_check(args["dtype_in"], args["dtype_out"], args["ta"], args["tb"], args["M"],
                           args["N"], args["K"], args["A"], args["lda"], args["sA"], args["B"],
                           args["ldb"], args["sB"], args["beta"], args["Cp"], args["ldc"], args["sC"],
                           args["batch"], C.byref(args["epi"]) if args["epi"] else None)
    return st, _lib.last_error()


def test_gemm_check_accepts_valid_layouts():
    assert _check()[0] == _lib.IT_OK
    assert _check(ta=1, lda=4)[0] == _lib.IT_OK          # A stored [K,M]
    assert _check(tb=1, ldb=6)[0] == _lib.IT_OK          # B stored [N,K]
    assert _check(M=0, Cp=None, A=None, B=None)[0] == _lib.IT_OK  # empty output
    assert _check(K=0, A=None, B=None)[0] == _lib.IT_OK  # C = 0 (+ epilogue)


def test_gemm_check_precision_mismatch():
    st, msg = _check(dtype_in=_lib.IT_F16)
    assert st == _lib.IT_ERR_PRECISION and "precision mismatch" in msg and "FP16" in msg
    st, _ = _check(dtype_out=7)
    assert st == _lib.IT_ERR_PRECISION


def test_gemm_check_bad_values():
    assert _check(ta=2)[0] == _lib.IT_ERR_INVALID
    assert _check(M=-1)[0] == _lib.IT_ERR_INVALID
    st, msg = _check(lda=5)
    assert st == _lib.IT_ERR_INVALID and "lda" in msg
    assert _check(ta=1, lda=3)[0] == _lib.IT_ERR_INVALID
    assert _check(ldb=4)[0] == _lib.IT_ERR_INVALID
    assert _check(ldc=4)[0] == _lib.IT_ERR_INVALID
    assert _check(sA=-1)[0] == _lib.IT_ERR_INVALID
    assert _check(Cp=None)[0] == _lib.IT_ERR_NULL
    assert _check(A=None)[0] == _lib.IT_ERR_NULL


def test_gemm_check_epilogues():
    epi = _lib.Epilogue(flags=0x80)
    assert _check(epi=epi)[0] == _lib.IT_ERR_INVALID
    epi = _lib.Epilogue(flags=_lib.IT_EPI_BIAS)
    assert _check(epi=epi)[0] == _lib.IT_ERR_NULL
    epi = _lib.Epilogue(flags=_lib.IT_EPI_SWIGLU, B2=16)
    assert _check(epi=epi)[0] == _lib.IT_ERR_INVALID          # needs NT
    assert _check(epi=epi, tb=1, ldb=6)[0] == _lib.IT_OK
    assert _check(epi=epi, tb=1, ldb=6, beta=1.0)[0] == _lib.IT_ERR_INVALID
    epi = _lib.Epilogue(flags=_lib.IT_EPI_CAUSAL)
    assert _check(epi=epi)[0] == _lib.IT_OK
    assert _check(epi=epi, beta=2.0)[0] == _lib.IT_ERR_INVALID


def test_gemm_rejects_before_device_work():
    lib = _lib.load()
    st = lib.it_gemm(None, _lib.IT_F16, _lib.IT_F32, 0, 0, 2, 2, 2, 1.0, 16, 2, 0, 16, 2, 0, 0.0,
                     16, 2, 0, 1, None)
    assert st == _lib.IT_ERR_PRECISION
    st = lib.it_gemm(None, _lib.IT_F32, _lib.IT_F32, 0, 0, 2, 2, 2, 1.0, 16, 2, 0, 16, 2, 0, 0.0,
                     16, 2, 0, 1, None)
    assert st == _lib.IT_ERR_NULL and "ctx" in _lib.last_error()


def test_gemm_group_validates_every_call_first():
    """it_gemm_group checks its count and each call as it_gemm does before touching the context
    (a NULL context is reported only once every call is valid)."""
    lib = _lib.load()
    arr = (_lib.GemmCall * 9)()
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 9, arr)
    assert st == _lib.IT_ERR_INVALID and "count" in _lib.last_error()
    assert lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, None) == _lib.IT_ERR_NULL
    good = _lib.GemmCall(_lib.IT_OP_T, _lib.IT_OP_N, 4, 4, 4, 1.0, 16, 4, 0, 16, 4, 0, 0.0, 16, 4, 0, 1, None)
    bad = _lib.GemmCall(_lib.IT_OP_T, _lib.IT_OP_N, 4, 4, 4, 1.0, 16, 2, 0, 16, 4, 0, 0.0, 16, 4, 0, 1, None)
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, (_lib.GemmCall * 2)(good, bad))
    assert st == _lib.IT_ERR_INVALID and "lda" in _lib.last_error()
    other = _lib.GemmCall(_lib.IT_OP_T, _lib.IT_OP_N, 4, 4, 4, 1.0, 4096, 4, 0, 8192, 4, 0, 0.0, 12288, 4, 0, 1,
                          None)
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, (_lib.GemmCall * 2)(good, other))
    assert st == _lib.IT_ERR_NULL and "ctx" in _lib.last_error()
    # One call's output may not overlap another call's operands or output (the group may run them
    # in one launch): the same buffers twice, and an output that lands inside the next call's B.
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, (_lib.GemmCall * 2)(good, good))
    assert st == _lib.IT_ERR_INVALID and "overlaps" in _lib.last_error()
    into_b = _lib.GemmCall(_lib.IT_OP_T, _lib.IT_OP_N, 4, 4, 4, 1.0, 4096, 4, 0, 8192, 4, 0, 0.0, 8200, 4, 0, 1, None)
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, (_lib.GemmCall * 2)(other, into_b))
    assert st == _lib.IT_ERR_INVALID and "call 1 overlaps the operands or outputs of call 0" in _lib.last_error()
    st = lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 2, (_lib.GemmCall * 2)(other, _lib.GemmCall(
        _lib.IT_OP_T, _lib.IT_OP_N, 4, 4, 4, 1.0, 4096, 4, 0, 8192, 4, 0, 0.0, 12288 + 64, 4, 0, 1, None)))
    assert st == _lib.IT_ERR_NULL  # C ranges [12288, 12352) and [12352, 12416) only touch
    assert lib.it_gemm_group(None, _lib.IT_BF16, _lib.IT_F32, 0, None) == _lib.IT_ERR_NULL  # ctx checked last


def test_null_context_calls_fail_cleanly():
    lib = _lib.load()
    assert lib.it_malloc(None, 16, C.byref(C.c_void_p())) == _lib.IT_ERR_NULL
    assert lib.it_stream_sync(None) == _lib.IT_ERR_NULL
    assert lib.it_mem_allocated(None) == 0
    assert lib.it_attention_forward(None, _lib.IT_F32, 1, 1, 1, 1, 1.0, 0, None, None, None,
                                    None, None, None, None, None, None) == _lib.IT_ERR_NULL


def test_init_without_device_reports_no_device():
    lib = _lib.load()
    if lib.it_device_count() > 0:
        pytest.skip("a device is visible; the no-device path is exercised on CPU-only hosts")
    h = C.c_void_p()
    assert lib.it_init(0, C.byref(h)) == _lib.IT_ERR_NO_DEVICE
    assert "no HIP device" in _lib.last_error()


# ------------------------------------------------------------------ host mirror errors (no device)

class _NoDevice:
    """Stands in for a device buffer so shape/precision checks can run without a GPU."""
    ptr = 0
    ctx = None


def _t(shape, prec=Precision.FP32):
    return Tensor(_NoDevice(), shape, prec)


def test_mirror_matmul_errors_match_reference():
    import irontensor_amd as it
    with pytest.raises(it.PrecisionMismatch, match="matmul: precision mismatch, expected FP32, got BF16"):
        it.matmul(_t([2, 2], Precision.BF16), _t([2, 2]))
    with pytest.raises(it.UnsupportedDimensions, match=r"expected 2D or 3D tensors, got \[4, 4\]"):
        it.matmul(_t([1, 1, 2, 2]), _t([1, 1, 2, 2]))
    with pytest.raises(it.InnerDimensionMismatch, match=r"A=\[2, 3\], B=\[4, 5\]"):
        it.matmul(_t([2, 3]), _t([4, 5]))
    with pytest.raises(it.ShapeMismatch, match="expected batch size 2, got batch size 3"):
        it.matmul(_t([2, 3, 4]), _t([3, 4, 5]))
    with pytest.raises(it.InnerDimensionMismatch, match="matmul_batched"):
        it.matmul(_t([2, 3, 4]), _t([2, 5, 5]))


def test_mirror_panics_match_reference():
    import irontensor_amd as it
    with pytest.raises(it.Panic, match=r"Inner dimensions must match: A\[4, 3\] @ B\[5, 2\]\^T"):
        it.matmul_mps_nt(_t([4, 3]), _t([5, 2]))
    with pytest.raises(it.Panic, match=r"Inner dimensions must match: A\[3, 4\]\^T @ B\[2, 5\]"):
        it.matmul_mps_tn(_t([3, 4]), _t([2, 5]))
    with pytest.raises(it.Panic, match="requires 2D"):
        it.matmul_mps_nt(_t([1, 4, 3]), _t([5, 3]))
    with pytest.raises(it.Panic, match="only supports FP32"):
        it.matmul_mps_tn(_t([3, 4], Precision.BF16), _t([3, 5]))
    with pytest.raises(it.Panic, match="matmul_bf16 requires BF16 input A"):
        it.matmul_bf16(_t([2, 3]), _t([3, 2], Precision.BF16))
    with pytest.raises(it.Panic, match="Q must be 4D"):
        it.attention(_t([2, 3, 4]), _t([1, 2, 3, 4]), _t([1, 2, 3, 4]), True)
    with pytest.raises(it.Panic, match="requires 2D, 3D, or 4D"):
        it.matmul_backward(_t([2]), _t([2]), _t([2]))
    with pytest.raises(it.Panic, match="Data length 3 does not match shape"):
        it.Tensor.from_f32_slice([1, 2, 3], [2, 2])


def test_error_display_formats():
    import irontensor_amd as it
    # src/error.rs:43-66
    assert str(it.ShapeMismatch("op", "a", "b")) == "op: shape mismatch, expected a, got b"
    assert str(it.UnsupportedDimensions("op", "2D", [1, 2])) == "op: unsupported dimensions, expected 2D, got [1, 2]"
    assert str(it.PrecisionMismatch("op", "FP32", "BF16")) == "op: precision mismatch, expected FP32, got BF16"
    assert str(it.InnerDimensionMismatch("op", [1, 2], [3, 4])) == "op: inner dimensions don't match, A=[1, 2], B=[3, 4]"
    assert str(it.EmptyTensor("op")) == "op: empty tensor not supported"
    assert str(it.InvalidValue("op", "bad")) == "op: bad"


def test_noalloc_backward_refuses_sizes_beyond_its_static_workspace():
    """it_flash_attention_backward_noalloc keeps two floats per query row in an 8 MiB static device array:
    more than 1048576 query rows (bh * seq) are refused on the host, before the context or any
    buffer is looked at (so no device is needed here)."""
    lib = _lib.load()
    lay = _lib.AttnLayout(1, 0, 0, 64)
    ptrs = [C.c_void_p(256)] * 9

    def call(bh, seq):
        return lib.it_flash_attention_backward_noalloc(None, _lib.IT_BF16, bh, seq, 64, C.c_float(0.125), 1,
                                                       C.byref(lay), None, None, *ptrs)

    assert call(1025, 1024) == _lib.IT_ERR_DIMS
    assert "static workspace" in _lib.last_error()
    assert call(1, 1048577) == _lib.IT_ERR_DIMS
    assert call(1024, 1024) == _lib.IT_ERR_NULL  # within the limit: the NULL context is the next refusal
