"""ctypes wrapper of the CPU oracle (oracle/liboracle.so) -- TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may use this package, and only
as the checker / the timed CPU baseline. The product (irontensor_amd) never imports it.
"""
from __future__ import annotations

import ctypes as C
import os
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"

_lib = None


def build() -> Path:
    """Compiles liboracle.so with gcc (oracle/Makefile)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load() -> C.CDLL:
    global _lib
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        build()
    lib = C.CDLL(str(LIB_PATH))
    vp, i64, i = C.c_void_p, C.c_int64, C.c_int
    lib.ref_f32_to_bf16.restype = C.c_uint16
    lib.ref_f32_to_bf16.argtypes = [C.c_float]
    lib.ref_bf16_to_f32.restype = C.c_float
    lib.ref_bf16_to_f32.argtypes = [C.c_uint16]
    lib.ref_f32_to_bf16_n.argtypes = [vp, vp, i64]
    lib.ref_bf16_to_f32_n.argtypes = [vp, vp, i64]
    gemm_args = [i, i, i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i64, i64, i64, i]
    lib.ref_gemm_f32.argtypes = gemm_args
    lib.ref_gemm_f64.argtypes = gemm_args
    lib.ref_gemm_bf16.argtypes = [i, i, i64, i64, i64, vp, i64, i64, vp, i64, i64, vp, i, i64, i64,
                                  i64, i]
    lib.ref_add_bias.argtypes = [vp, vp, i64, i64]
    lib.ref_swiglu.argtypes = [vp, vp, vp, i64]
    lib.ref_swiglu_backward.argtypes = [vp, vp, vp, vp, vp, i64]
    lib.ref_softmax_rows.argtypes = [vp, i64, i64]
    lib.ref_softmax_backward.argtypes = [vp, vp, vp, i64, i64]
    lib.ref_attention_bshd.argtypes = [vp, vp, vp, vp, i64, i64, i64, i64, i, i]
    lib.ref_attention_fwd_bhsd.argtypes = [vp, vp, vp, vp, vp, i64, i64, i64, C.c_float, i, i]
    lib.ref_attention_bwd_bhsd.argtypes = [vp, vp, vp, vp, vp, vp, vp, i64, i64, i64, C.c_float, i, i]
    lib.ref_default_threads.restype = i
    lib.ref_transpose_3d.argtypes = [vp, vp, i64, i64, i64]
    lib.ref_causal_mask_3d.argtypes = [vp, vp, i64, i64]
    f = C.c_float
    lib.ref_rmsnorm_forward.argtypes = [vp, vp, vp, i64, i64, f]
    lib.ref_rmsnorm_backward.argtypes = [vp, vp, vp, vp, vp, i64, i64, f]
    lib.ref_rope.argtypes = [vp, i64, i64, i64, i64, i64, f, i64, i]
    lib.ref_embedding_forward.argtypes = [vp, vp, vp, i64, i64]
    lib.ref_embedding_backward.argtypes = [vp, vp, vp, i64, i64, i64]
    lib.ref_cross_entropy.argtypes = [vp, vp, vp, vp, i64, i64]
    lib.ref_cross_entropy.restype = f
    lib.ref_lion.argtypes = [vp, vp, vp, i64, f, f, f, f, f]
    lib.ref_sum_squares.argtypes = [vp, i64]
    lib.ref_sum_squares.restype = C.c_double
    lib.ref_fused_rmsnorm_linear.argtypes = [vp, vp, vp, vp, i64, i64, i64, f]
    lib.ref_fused_linear_cross_entropy.argtypes = [vp, vp, vp, vp, vp, vp, i64, i64, i64]
    lib.ref_fused_linear_cross_entropy.restype = C.c_float
    _lib = lib
    return lib


def default_threads() -> int:
    env = os.environ.get("ORACLE_THREADS")
    if env:
        return max(1, int(env))
    return min(16, int(load().ref_default_threads()))


def _p(a: np.ndarray):
    return a.ctypes.data_as(C.c_void_p)


def _c(a, dtype) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=dtype)


def _gemm_dims(a: np.ndarray, b: np.ndarray, trans_a: bool, trans_b: bool):
    batched = a.ndim == 3
    batch = a.shape[0] if batched else 1
    ra, ca = a.shape[-2:]
    rb, cb = b.shape[-2:]
    m, k = (ca, ra) if trans_a else (ra, ca)
    k2, n = (cb, rb) if trans_b else (rb, cb)
    assert k == k2, (a.shape, b.shape, trans_a, trans_b)
    s_a = ra * ca if batched else 0
    s_b = rb * cb if b.ndim == 3 else 0
    return batched, batch, m, n, k, ca, cb, s_a, s_b


def gemm_f32(a, b, trans_a=False, trans_b=False, threads=None) -> np.ndarray:
    """op(A).op(B) with the reference's sequential f32 loop (2D, or 3D batched)."""
    a, b = _c(a, np.float32), _c(b, np.float32)
    batched, batch, m, n, k, lda, ldb, s_a, s_b = _gemm_dims(a, b, trans_a, trans_b)
    out = np.empty((batch, m, n) if batched else (m, n), dtype=np.float32)
    load().ref_gemm_f32(int(trans_a), int(trans_b), m, n, k, _p(a), lda, s_a, _p(b), ldb, s_b,
                        _p(out), n, m * n, batch, threads or default_threads())
    return out


def gemm_f64(a, b, trans_a=False, trans_b=False, threads=None) -> np.ndarray:
    a, b = _c(a, np.float32), _c(b, np.float32)
    batched, batch, m, n, k, lda, ldb, s_a, s_b = _gemm_dims(a, b, trans_a, trans_b)
    out = np.empty((batch, m, n) if batched else (m, n), dtype=np.float64)
    load().ref_gemm_f64(int(trans_a), int(trans_b), m, n, k, _p(a), lda, s_a, _p(b), ldb, s_b,
                        _p(out), n, m * n, batch, threads or default_threads())
    return out


def gemm_bf16(a_u16, b_u16, trans_a=False, trans_b=False, out_bf16=False, threads=None) -> np.ndarray:
    a, b = _c(a_u16, np.uint16), _c(b_u16, np.uint16)
    batched, batch, m, n, k, lda, ldb, s_a, s_b = _gemm_dims(a, b, trans_a, trans_b)
    shape = (batch, m, n) if batched else (m, n)
    out = np.empty(shape, dtype=np.uint16 if out_bf16 else np.float32)
    load().ref_gemm_bf16(int(trans_a), int(trans_b), m, n, k, _p(a), lda, s_a, _p(b), ldb, s_b,
                         _p(out), int(out_bf16), n, m * n, batch, threads or default_threads())
    return out


def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    out = np.empty(x.shape, dtype=np.uint16)
    load().ref_f32_to_bf16_n(_p(x), _p(out), x.size)
    return out


def bf16_to_f32(x) -> np.ndarray:
    x = _c(x, np.uint16)
    out = np.empty(x.shape, dtype=np.float32)
    load().ref_bf16_to_f32_n(_p(x), _p(out), x.size)
    return out


def add_bias(y, bias) -> np.ndarray:
    y = _c(y, np.float32).copy()
    bias = _c(bias, np.float32)
    load().ref_add_bias(_p(y), _p(bias), y.shape[0], y.shape[1])
    return y


def swiglu(gate, up) -> np.ndarray:
    g, u = _c(gate, np.float32), _c(up, np.float32)
    out = np.empty_like(g)
    load().ref_swiglu(_p(g), _p(u), _p(out), g.size)
    return out


def swiglu_backward(grad_out, gate, up):
    go, g, u = _c(grad_out, np.float32), _c(gate, np.float32), _c(up, np.float32)
    gg, gu = np.empty_like(g), np.empty_like(g)
    load().ref_swiglu_backward(_p(go), _p(g), _p(u), _p(gg), _p(gu), g.size)
    return gg, gu


def softmax_rows(x) -> np.ndarray:
    x = _c(x, np.float32).copy()
    cols = x.shape[-1]
    load().ref_softmax_rows(_p(x), x.size // cols, cols)
    return x


def softmax_backward(grad_y, y) -> np.ndarray:
    gy, yy = _c(grad_y, np.float32), _c(y, np.float32)
    out = np.empty_like(yy)
    cols = yy.shape[-1]
    load().ref_softmax_backward(_p(gy), _p(yy), _p(out), yy.size // cols, cols)
    return out


def attention_bshd(q, k, v, causal: bool, threads=None) -> np.ndarray:
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    b, s, h, d = q.shape
    out = np.empty_like(q)
    load().ref_attention_bshd(_p(q), _p(k), _p(v), _p(out), b, s, h, d, int(causal),
                              threads or default_threads())
    return out


def attention_fwd_bhsd(q, k, v, scale: float, causal: bool, threads=None):
    """q, k, v: [BH, S, D] (or [B,H,S,D]); returns (O, P)."""
    q, k, v = _c(q, np.float32), _c(k, np.float32), _c(v, np.float32)
    s, d = q.shape[-2:]
    bh = q.size // (s * d)
    out = np.empty_like(q)
    p = np.empty((bh, s, s), dtype=np.float32)
    load().ref_attention_fwd_bhsd(_p(q), _p(k), _p(v), _p(out), _p(p), bh, s, d, float(scale),
                                  int(causal), threads or default_threads())
    return out, p


def attention_bwd_bhsd(d_o, q, k, v, scale: float, causal: bool, threads=None):
    """Returns (dQ, dK, dV) in the shape of q."""
    d_o, q, k, v = (_c(t, np.float32) for t in (d_o, q, k, v))
    s, d = q.shape[-2:]
    bh = q.size // (s * d)
    dq, dk, dv = np.empty_like(q), np.empty_like(q), np.empty_like(q)
    load().ref_attention_bwd_bhsd(_p(d_o), _p(q), _p(k), _p(v), _p(dq), _p(dk), _p(dv), bh, s, d,
                                  float(scale), int(causal), threads or default_threads())
    return dq, dk, dv


def transpose_3d(x, batch: int, m: int, n: int) -> np.ndarray:
    """[batch, m, n] -> [batch, n, m] (transpose_3d_f32, src/shaders/attention.metal:163-182)."""
    x = _c(x, np.float32)
    assert x.size == batch * m * n
    out = np.empty((batch, n, m), np.float32)
    load().ref_transpose_3d(_p(x), _p(out), batch, m, n)
    return out


def causal_mask_3d(x, batch: int, seq: int) -> np.ndarray:
    """columns > row set to -inf over [batch, seq, seq] (causal_mask_3d_f32, attention.metal:186-207)."""
    x = _c(x, np.float32)
    assert x.size == batch * seq * seq
    out = np.empty((batch, seq, seq), np.float32)
    load().ref_causal_mask_3d(_p(x), _p(out), batch, seq)
    return out


# ---------------------------------------------------------------- training-step ops (train_ref.c)

def rmsnorm(x, gamma, eps: float = 1e-5) -> np.ndarray:
    x, g = _c(x, np.float32), _c(gamma, np.float32)
    dim = x.shape[-1]
    y = np.empty_like(x)
    load().ref_rmsnorm_forward(_p(x), _p(g), _p(y), x.size // dim, dim, float(eps))
    return y


def rmsnorm_backward(dy, x, gamma, eps: float = 1e-5):
    dy, x, g = _c(dy, np.float32), _c(x, np.float32), _c(gamma, np.float32)
    dim = x.shape[-1]
    dx, dg = np.empty_like(x), np.empty(dim, np.float32)
    load().ref_rmsnorm_backward(_p(dy), _p(x), _p(g), _p(dx), _p(dg), x.size // dim, dim, float(eps))
    return dx, dg


def rope(x, base: float = 10000.0, offset: int = 0, backward: bool = False, heads=None, head_dim=None):
    """x: [batch, seq, heads, head_dim] (or [batch, seq, cols] with heads*head_dim <= cols and the
    rotated block at column 0); returns a rotated copy."""
    y = _c(x, np.float32).copy()
    if y.ndim == 4:
        b, s, h, d = y.shape
        rs = h * d
    else:
        b, s, rs = y.shape
        h, d = heads, head_dim
    load().ref_rope(_p(y), b, s, h, d, rs, float(base), int(offset), int(backward))
    return y


def embedding(table, ids) -> np.ndarray:
    t, ids = _c(table, np.float32), _c(ids, np.uint32)
    out = np.empty((ids.size, t.shape[1]), np.float32)
    load().ref_embedding_forward(_p(t), _p(ids), _p(out), ids.size, t.shape[1])
    return out


def embedding_backward(dy, ids, vocab: int) -> np.ndarray:
    dy, ids = _c(dy, np.float32), _c(ids, np.uint32)
    dw = np.empty((vocab, dy.shape[1]), np.float32)
    load().ref_embedding_backward(_p(dy), _p(ids), _p(dw), ids.size, dy.shape[1], vocab)
    return dw


def cross_entropy(logits, targets):
    """Returns (mean_loss, per-row losses, grad_logits)."""
    x, t = _c(logits, np.float32), _c(targets, np.uint32)
    rows, vocab = x.shape
    losses, grad = np.empty(rows, np.float32), np.empty_like(x)
    mean = load().ref_cross_entropy(_p(x), _p(t), _p(losses), _p(grad), rows, vocab)
    return float(np.float32(mean)), losses, grad


def lion(w, m, g, lr: float, beta1: float, beta2: float, wd: float, scale: float = 1.0):
    """Returns updated copies (w, m)."""
    w, m, g = _c(w, np.float32).copy(), _c(m, np.float32).copy(), _c(g, np.float32)
    load().ref_lion(_p(w), _p(m), _p(g), w.size, float(lr), float(beta1), float(beta2), float(wd), float(scale))
    return w, m


def sum_squares(x) -> float:
    x = _c(x, np.float32)
    return float(load().ref_sum_squares(_p(x), x.size))


def fused_rmsnorm_linear(x, gamma, w, eps: float = 1e-5) -> np.ndarray:
    x, g, w = _c(x, np.float32), _c(gamma, np.float32), _c(w, np.float32)
    rows, hidden = x.shape
    out = np.empty((rows, w.shape[0]), np.float32)
    load().ref_fused_rmsnorm_linear(_p(x), _p(g), _p(w), _p(out), rows, hidden, w.shape[0], float(eps))
    return out


def fused_linear_cross_entropy(hidden, weight, targets, with_weight_grad: bool = True):
    """Returns (mean loss over valid targets, per-row losses, grad_hidden, grad_weight or None).
    targets are int32; values outside [0, vocab) (-100 by convention) are ignored."""
    h, w = _c(hidden, np.float32), _c(weight, np.float32)
    t = _c(targets, np.int32)
    rows, hd = h.shape
    vocab = w.shape[0]
    losses, gh = np.empty(rows, np.float32), np.empty_like(h)
    gw = np.empty_like(w) if with_weight_grad else None
    mean = load().ref_fused_linear_cross_entropy(_p(h), _p(w), _p(t), _p(losses), _p(gh),
                                                 _p(gw) if gw is not None else None, rows, hd, vocab)
    return float(np.float32(mean)), losses, gh, gw
