"""The reference's matmul-path ops API, on the MI355X C ABI.

Same names, argument meaning and error behaviour as IronTensor's Rust functions (each docstring
cites the function it mirrors). Every op launches hand-written HIP through libirontensor_hip.so;
there is no CPU or library fallback.
"""
from __future__ import annotations

import ctypes as C
import math
from typing import Optional, Sequence, Tuple

from . import _lib
from .errors import (InnerDimensionMismatch, InvalidValue, Panic, PrecisionMismatch, ShapeMismatch,
                     UnsupportedDimensions, check)
from .tensor import Precision, Tensor

_P = Precision


def _vp(t: Optional[Tensor]):
    return C.c_void_p(t.ptr) if t is not None else C.c_void_p(0)


def _prec_name(p: Precision) -> str:
    return "BF16" if p is _P.BF16 else ("FP32" if p is _P.FP32 else "unknown")


def gemm(a: Tensor, b: Tensor, *, trans_a: bool = False, trans_b: bool = False, alpha: float = 1.0,
         beta: float = 0.0, out: Optional[Tensor] = None, out_precision: Optional[Precision] = None,
         bias: Optional[Tensor] = None, causal: bool = False, causal_offset: int = 0,
         b2: Optional[Tensor] = None, gate_out: Optional[Tensor] = None,
         up_out: Optional[Tensor] = None, op: str = "matmul") -> Tensor:
    """C = alpha * op(A) . op(B) + beta * C with the fused epilogues, 2D or 3D (batched).

    This is the general entry the named ops below reduce to (it_gemm). op(A) is A or A^T of the
    last two dims; batch dims must match (or be absent on B, which then broadcasts).
    """
    if a.precision() != b.precision():
        raise PrecisionMismatch(op, _prec_name(a.precision()), _prec_name(b.precision()))
    sa, sb = a.shape(), b.shape()
    if len(sa) not in (2, 3) or len(sb) not in (2, 3) or (len(sa) == 2 and len(sb) == 3):
        raise UnsupportedDimensions(op, "2D or 3D tensors", [len(sa), len(sb)])
    batch = sa[0] if len(sa) == 3 else 1
    if len(sb) == 3 and sb[0] != batch:
        raise ShapeMismatch(op, f"batch size {batch}", f"batch size {sb[0]}")
    ra, ca = sa[-2], sa[-1]
    rb, cb = sb[-2], sb[-1]
    M, K = (ca, ra) if trans_a else (ra, ca)
    K2, N = (cb, rb) if trans_b else (rb, cb)
    if K != K2:
        raise InnerDimensionMismatch(op, sa, sb)
    out_prec = out_precision if out_precision is not None else _P.FP32
    out_shape = [batch, M, N] if len(sa) == 3 else [M, N]
    if out is None:
        out = Tensor.empty(out_shape, out_prec, a.ctx)
        if beta != 0.0:
            raise Panic("beta != 0 needs an explicit output tensor")
    elif out.shape() != out_shape:
        raise ShapeMismatch(op, str(out_shape), str(out.shape()))
    epi = _lib.Epilogue()
    use_epi = False
    if bias is not None:
        epi.flags |= _lib.IT_EPI_BIAS
        epi.bias = bias.ptr
        use_epi = True
    if b2 is not None:
        epi.flags |= _lib.IT_EPI_SWIGLU
        epi.B2 = b2.ptr
        epi.gate_out = gate_out.ptr if gate_out is not None else None
        epi.up_out = up_out.ptr if up_out is not None else None
        use_epi = True
    if causal:
        epi.flags |= _lib.IT_EPI_CAUSAL
        epi.causal_offset = causal_offset
        use_epi = True
    lib = a.ctx.lib
    st = lib.it_gemm(a.ctx.handle, int(a.precision()), int(out.precision()),
                     _lib.IT_OP_T if trans_a else _lib.IT_OP_N,
                     _lib.IT_OP_T if trans_b else _lib.IT_OP_N,
                     M, N, K, float(alpha),
                     _vp(a), ca, ra * ca if len(sa) == 3 else 0,
                     _vp(b), cb, rb * cb if len(sb) == 3 else 0,
                     float(beta), _vp(out), N, M * N if len(sa) == 3 else 0, batch,
                     C.byref(epi) if use_epi else None)
    check(st, op)
    return out


def gemm_group(calls, op: str = "matmul_group") -> None:
    """Several independent 2D GEMMs in one it_gemm_group call: `calls` holds up to 8 tuples
    (a, b, out, trans_a, trans_b), out = op(a) . op(b), all of one input and one output precision.
    Calls of one layout run as one launch where the library can (BF16: whole 256 x 256 tiles in
    one round; FP32: 64 x 64 tiles with one split count for the group and one grouped reduction,
    when that is priced below the separate plans); otherwise as separate GEMMs. No counterpart in the reference (its command batch issues each
    GEMM separately); for callers holding several GEMMs at once, such as a layer's weight
    gradients."""
    if not calls:
        return
    if len(calls) > 8:
        raise Panic(f"{op}: at most 8 GEMMs per group, got {len(calls)}")
    a0, _, o0, _, _ = calls[0]
    structs = []
    for a, b, out, ta, tb in calls:
        if a.precision() != a0.precision() or b.precision() != a0.precision():
            raise PrecisionMismatch(op, _prec_name(a0.precision()), _prec_name(b.precision()))
        if out.precision() != o0.precision():
            raise PrecisionMismatch(op, _prec_name(o0.precision()), _prec_name(out.precision()))
        sa, sb = a.shape(), b.shape()
        if len(sa) != 2 or len(sb) != 2:
            raise UnsupportedDimensions(op, "2D tensors", [len(sa), len(sb)])
        M, K = (sa[1], sa[0]) if ta else (sa[0], sa[1])
        K2, N = (sb[1], sb[0]) if tb else (sb[0], sb[1])
        if K != K2:
            raise InnerDimensionMismatch(op, sa, sb)
        if out.shape() != [M, N]:
            raise ShapeMismatch(op, str([M, N]), str(out.shape()))
        structs.append(_lib.GemmCall(_lib.IT_OP_T if ta else _lib.IT_OP_N, _lib.IT_OP_T if tb else _lib.IT_OP_N,
                                     M, N, K, 1.0, a.ptr, sa[1], 0, b.ptr, sb[1], 0, 0.0, out.ptr, N, 0, 1, None))
    arr = (_lib.GemmCall * len(structs))(*structs)
    check(a0.ctx.lib.it_gemm_group(a0.ctx.handle, int(a0.precision()), int(o0.precision()), len(structs), arr), op)


# ------------------------------------------------------------------ FP32 matmul family

def matmul_mps(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/mps_gemm.rs:44-91: C = A.B, FP32, 2D [M,K].[K,N] or 3D batched; TensorError on
    precision (:45-58), rank (:77-81), inner dim (:102-108, :446-451) and batch (:439-445)."""
    for t in (a, b):
        if t.precision() is not _P.FP32:
            raise PrecisionMismatch("matmul", "FP32", "BF16" if t.precision() is _P.BF16 else "unknown")
    sa, sb = a.shape(), b.shape()
    if (len(sa), len(sb)) == (2, 2):
        if sa[1] != sb[0]:
            raise InnerDimensionMismatch("matmul", sa, sb)
        return gemm(a, b)
    if (len(sa), len(sb)) == (3, 3):
        if sa[0] != sb[0]:
            raise ShapeMismatch("matmul_batched", f"batch size {sa[0]}", f"batch size {sb[0]}")
        if sa[2] != sb[1]:
            raise InnerDimensionMismatch("matmul_batched", sa, sb)
        return gemm(a, b, op="matmul_batched")
    raise UnsupportedDimensions("matmul", "2D or 3D tensors", [len(sa), len(sb)])


def matmul(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/gemm.rs:88-91 (delegates to matmul_mps)."""
    return matmul_mps(a, b)


def _assert_f32_2d(a: Tensor, b: Tensor, name: str) -> None:
    if a.precision() is not _P.FP32 or b.precision() is not _P.FP32:
        raise Panic("MPS matmul currently only supports FP32")
    if len(a.shape()) != 2 or len(b.shape()) != 2:
        raise Panic(f"{name} requires 2D tensors")


def matmul_mps_nt(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/mps_gemm.rs:213-314: Y = A.B^T with A [M,K], B [N,K]; panics on mismatch."""
    _assert_f32_2d(a, b, "matmul_mps_nt")
    (m, k), (n, k2) = a.shape(), b.shape()
    if k != k2:
        raise Panic(f"Inner dimensions must match: A[{m}, {k}] @ B[{n}, {k2}]^T")
    return gemm(a, b, trans_b=True, op="matmul_mps_nt")


def matmul_mps_tn(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/mps_gemm.rs:325-426: C = A^T.B with A [K,M], B [K,N]; panics on mismatch."""
    _assert_f32_2d(a, b, "matmul_mps_tn")
    (k, m), (k2, n) = a.shape(), b.shape()
    if k != k2:
        raise Panic(f"Inner dimensions must match: A[{k}, {m}]^T @ B[{k2}, {n}]")
    return gemm(a, b, trans_a=True, op="matmul_mps_tn")


def matmul_custom(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/gemm.rs:102-285 (the custom-kernel path): same contract as matmul, panicking."""
    try:
        return matmul_mps(a, b)
    except (PrecisionMismatch, UnsupportedDimensions, InnerDimensionMismatch, ShapeMismatch) as e:
        raise Panic(str(e)) from e


def matmul_tn(a: Tensor, b: Tensor) -> Tensor:
    """src/train/helpers.rs:80-83 and src/train/trainer/train_step.rs:20-22."""
    return matmul_mps_tn(a, b)


def matmul_backward_a(grad_c: Tensor, b: Tensor) -> Tensor:
    """src/ops/backward/gemm.rs:106-133: grad_A = grad_C . B^T (NT), 2D or 3D."""
    if grad_c.precision() is not _P.FP32 or b.precision() is not _P.FP32:
        raise Panic("matmul_backward_a requires FP32")
    g, s = grad_c.shape(), b.shape()
    if len(g) == 2 and len(s) == 2:
        if s[1] != g[1]:
            raise Panic(f"assertion `left == right` failed: {s[1]} != {g[1]}")
    elif len(g) == 3 and len(s) == 3:
        if s[0] != g[0] or s[2] != g[2]:
            raise Panic("assertion `left == right` failed")
    else:
        raise Panic("Unsupported shapes for matmul_backward_a")
    return gemm(grad_c, b, trans_b=True, op="matmul_backward_a")


def matmul_backward_b(grad_c: Tensor, a: Tensor) -> Tensor:
    """src/ops/backward/gemm.rs:136-163: grad_B = A^T . grad_C (TN), 2D or 3D."""
    if grad_c.precision() is not _P.FP32 or a.precision() is not _P.FP32:
        raise Panic("matmul_backward_b requires FP32")
    g, s = grad_c.shape(), a.shape()
    if len(g) == 2 and len(s) == 2:
        if s[0] != g[0]:
            raise Panic(f"assertion `left == right` failed: {s[0]} != {g[0]}")
    elif len(g) == 3 and len(s) == 3:
        if s[0] != g[0] or s[1] != g[1]:
            raise Panic("assertion `left == right` failed")
    else:
        raise Panic("Unsupported shapes for matmul_backward_b")
    return gemm(a, grad_c, trans_a=True, op="matmul_backward_b")


def matmul_backward(grad_c: Tensor, a: Tensor, b: Tensor) -> Tuple[Tensor, Tensor]:
    """src/ops/backward/gemm.rs:73-103: (grad_A, grad_B) for 2D, 3D, or 4D (leading dims collapsed)."""
    for t in (grad_c, a, b):
        if t.precision() is not _P.FP32:
            raise Panic("assertion `left == right` failed: precision")
    sa, sb = a.shape(), b.shape()
    if len(sa) == 4 and len(sb) == 4:
        bt = sa[0] * sa[1]
        ga, gb = matmul_backward(grad_c.view([bt] + grad_c.shape()[2:]), a.view([bt] + sa[2:]),
                                 b.view([bt] + sb[2:]))
        return ga.view(sa), gb.view(sb)
    if (len(sa), len(sb)) not in ((2, 2), (3, 3)):
        raise Panic(f"matmul_backward requires 2D, 3D, or 4D tensors, got shapes {sa} and {sb}")
    return matmul_backward_a(grad_c, b), matmul_backward_b(grad_c, a)


# ------------------------------------------------------------------ BF16

def to_bf16_gpu(t: Tensor) -> Tensor:
    """src/ops/bf16_ops/precision.rs:15-46 (RNE on the GPU)."""
    if t.precision() is _P.BF16:
        return t.clone()
    out = Tensor.empty(t.shape(), _P.BF16, t.ctx)
    check(t.ctx.lib.it_f32_to_bf16(t.ctx.handle, _vp(t), _vp(out), t.numel()), "to_bf16_gpu")
    return out


def to_f32_gpu(t: Tensor) -> Tensor:
    """src/ops/bf16_ops/precision.rs:48-78."""
    if t.precision() is _P.FP32:
        return t.clone()
    out = Tensor.empty(t.shape(), _P.FP32, t.ctx)
    check(t.ctx.lib.it_bf16_to_f32(t.ctx.handle, _vp(t), _vp(out), t.numel()), "to_f32_gpu")
    return out


def matmul_bf16(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/bf16_ops/gemm.rs:25-82: BF16 [M,K].[K,N] -> BF16, FP32 accumulation."""
    if a.precision() is not _P.BF16:
        raise Panic("matmul_bf16 requires BF16 input A")
    if b.precision() is not _P.BF16:
        raise Panic("matmul_bf16 requires BF16 input B")
    if len(a.shape()) != 2 or len(b.shape()) != 2:
        raise Panic("matmul_bf16 requires 2D tensors")
    if a.shape()[1] != b.shape()[0]:
        raise Panic("Inner dimensions must match")
    return gemm(a, b, out_precision=_P.BF16, op="matmul_bf16")


def matmul_bf16_batched(a: Tensor, b: Tensor) -> Tensor:
    """src/ops/bf16_ops/gemm.rs:85-146: BF16 [B,M,K].[B,K,N] -> BF16."""
    if a.precision() is not _P.BF16 or b.precision() is not _P.BF16:
        raise Panic("assertion `left == right` failed: BF16")
    sa, sb = a.shape(), b.shape()
    if len(sa) != 3 or len(sb) != 3:
        raise Panic("batched matmul requires 3D tensors")
    if sa[0] != sb[0]:
        raise Panic("Batch dimensions must match")
    if sa[2] != sb[1]:
        raise Panic("Inner dimensions must match")
    return gemm(a, b, out_precision=_P.BF16, op="matmul_bf16_batched")


# ------------------------------------------------------------------ trainer GEMM API

def ensure_fp32(t: Tensor) -> Tensor:
    """src/train/helpers.rs:12-18."""
    return to_f32_gpu(t) if t.precision() is _P.BF16 else t


def linear_forward(input: Tensor, weight: Tensor) -> Tensor:
    """src/train/helpers.rs:48-53: input [T,in] . weight[out,in]^T (BF16 weights widened first)."""
    return matmul_mps_nt(input, ensure_fp32(weight))


def linear_backward(grad_output: Tensor, input: Tensor, weight: Tensor) -> Tuple[Tensor, Tensor]:
    """src/train/helpers.rs:61-76: (dX = dY.W (NN), dW = dY^T.X (TN))."""
    w = ensure_fp32(weight)
    return matmul(grad_output, w), matmul_tn(grad_output, input)


def linear(input: Tensor, weight: Tensor, bias: Optional[Tensor] = None) -> Tensor:
    """nn::Linear::forward (src/nn/linear.rs:87-145): y = x.W^T + b over [..., in] inputs, with the
    bias add fused into the GEMM epilogue instead of the reference's CPU pass (:8-18)."""
    shape = input.shape()
    if not shape:
        raise Panic("Input must have at least one dimension")
    out_f, in_f = weight.shape()
    if shape[-1] != in_f:
        raise Panic(f"Input last dimension {shape[-1]} doesn't match in_features {in_f}")
    x = ensure_fp32(input)
    w = ensure_fp32(weight)
    b = ensure_fp32(bias) if bias is not None else None
    rows = max(1, math.prod(shape[:-1]))
    y = gemm(x.view([rows, in_f]), w, trans_b=True, bias=b, op="linear")
    return y.view(shape[:-1] + [out_f]) if len(shape) > 2 else y


class Linear:
    """nn::Linear parameter holder (src/nn/linear.rs:20-86) with the fused forward above."""

    def __init__(self, weight: Tensor, bias: Optional[Tensor] = None):
        self.weight = weight
        self.bias = bias
        self.out_features, self.in_features = weight.shape()

    @staticmethod
    def from_weight(weight: Tensor, bias: Optional[Tensor] = None) -> "Linear":
        return Linear(weight, bias)

    def forward(self, input: Tensor) -> Tensor:
        return linear(input, self.weight, self.bias)

    def num_params(self) -> int:
        return self.weight.numel() + (self.bias.numel() if self.bias is not None else 0)


def swiglu_up(x: Tensor, w_gate: Tensor, w_up: Tensor, out_precision: Optional[Precision] = None,
              keep_pre_activations: bool = True,
              bias: Optional[Tensor] = None) -> Tuple[Tensor, Optional[Tensor], Optional[Tensor]]:
    """FFN up-projection with the fused SwiGLU epilogue: h = silu(x.Wg^T + bg) * (x.Wu^T + bu).

    Replaces the two linear_forward calls plus swiglu (src/train/forward.rs:166-172,
    src/ops/elementwise.rs:351-354, src/shaders/elementwise.metal:100-115), and with `bias` the two
    Linear biases (src/nn/linear.rs:8-18): an FP32 [2F] tensor, gate bias then up bias. Returns
    (h, gate, up); gate and up are the pre-activations the backward needs (src/train/cache.rs:23-27).
    """
    prec = out_precision if out_precision is not None else (
        _P.BF16 if x.precision() is _P.BF16 else _P.FP32)
    rows, _ = x.shape()
    f = w_gate.shape()[0]
    if w_up.shape() != w_gate.shape():
        raise ShapeMismatch("swiglu", str(w_gate.shape()), str(w_up.shape()))
    if bias is not None and (bias.numel() != 2 * f or bias.precision() is not _P.FP32):
        raise ShapeMismatch("swiglu", f"FP32 bias of {2 * f} elements", str(bias.shape()))
    g = Tensor.empty([rows, f], prec, x.ctx) if keep_pre_activations else None
    u = Tensor.empty([rows, f], prec, x.ctx) if keep_pre_activations else None
    h = gemm(x, w_gate, trans_b=True, b2=w_up, gate_out=g, up_out=u, out_precision=prec,
             bias=bias, op="swiglu")
    return h, g, u


# ------------------------------------------------------------------ attention contractions

def _layout_bshd(batch: int, seq: int, heads: int, dim: int) -> _lib.AttnLayout:
    return _lib.AttnLayout(heads, seq * heads * dim, dim, heads * dim)


def _layout_bhsd(seq: int, dim: int) -> _lib.AttnLayout:
    return _lib.AttnLayout(1, seq * dim, 0, dim)


def attention(q: Tensor, k: Tensor, v: Tensor, causal: bool) -> Tensor:
    """src/ops/attention.rs:286-377: softmax(Q.K^T/sqrt(D), causal) . V on [B,S,H,D] tensors.

    The reference transposes to [B,H,S,D], materialises K^T and copies through the CPU; here the
    two GEMMs address the [B,S,H,D] operands in place (strided per head) and the scale and causal
    mask are fused.
    """
    for t in (q, k, v):
        if t.precision() is not _P.FP32:
            raise Panic("assertion `left == right` failed: attention requires FP32")
    qs, ks, vs = q.shape(), k.shape(), v.shape()
    if len(qs) != 4:
        raise Panic("Q must be 4D [batch, seq, heads, dim]")
    if len(ks) != 4:
        raise Panic("K must be 4D [batch, seq, heads, dim]")
    if len(vs) != 4:
        raise Panic("V must be 4D [batch, seq, heads, dim]")
    b, sq, h, d = qs
    skv = ks[1]
    if ks[0] != b or vs[0] != b:
        raise Panic("Batch size mismatch")
    if ks[2] != h or vs[2] != h:
        raise Panic("Num heads mismatch")
    if ks[3] != d or vs[3] != d:
        raise Panic("Head dim mismatch")
    if vs[1] != skv:
        raise Panic("K and V seq_len must match")
    out = Tensor.empty([b, sq, h, d], _P.FP32, q.ctx)
    if b == 0 or sq == 0 or skv == 0:
        return Tensor.zeros([b, sq, h, d], _P.FP32, q.ctx)
    if causal and sq != skv:
        raise Panic("Causal attention requires Q and K to have same seq_len")
    bh = b * h
    sc = Tensor.empty([bh, sq, skv], _P.FP32, q.ctx)
    p = Tensor.empty([bh, sq, skv], _P.FP32, q.ctx)
    lq, lkv = _layout_bshd(b, sq, h, d), _layout_bshd(b, skv, h, d)
    st = q.ctx.lib.it_attention_forward(q.ctx.handle, _lib.IT_F32, bh, sq, skv, d,
                                        1.0 / math.sqrt(d), int(causal), C.byref(lq), C.byref(lkv),
                                        C.byref(lq), _vp(q), _vp(k), _vp(v), _vp(sc), _vp(p), _vp(out))
    check(st, "attention")
    return out


def attention_forward_bhsd(q: Tensor, k: Tensor, v: Tensor, causal: bool = True,
                           scale: Optional[float] = None) -> Tuple[Tensor, Tensor]:
    """Forward contractions on [B,H,S,D] (FP32 or BF16 operands). Returns (O f32, P)."""
    b, h, s, d = q.shape()
    prec = q.precision()
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    sc = Tensor.empty([b * h, s, s], _P.FP32, q.ctx)
    p = Tensor.empty([b * h, s, s], prec, q.ctx)
    o = Tensor.empty([b, h, s, d], _P.FP32, q.ctx)
    lay = _layout_bhsd(s, d)
    check(q.ctx.lib.it_attention_forward(q.ctx.handle, int(prec), b * h, s, s, d, float(scale),
                                         int(causal), C.byref(lay), None, None, _vp(q), _vp(k),
                                         _vp(v), _vp(sc), _vp(p), _vp(o)), "attention")
    return o, p


def attention_backward_recompute(grad_output: Tensor, q: Tensor, k: Tensor, v: Tensor,
                                 causal: bool = True,
                                 scale: Optional[float] = None) -> Tuple[Tensor, Tensor, Tensor]:
    """src/train/helpers.rs:120-193 on [B,H,S,D]: returns (dQ, dK, dV), FP32.

    Recomputes S and P, then the five GEMMs with the transposed operands selected at launch (no
    transpose kernels) and the scale folded into the dQ / dK epilogues. The reference always
    applies the causal mask; `causal=False` is an extension.
    """
    b, h, s, d = q.shape()
    prec = q.precision()
    for t in (grad_output, k, v):
        if t.precision() is not prec:
            raise PrecisionMismatch("attention_backward", _prec_name(prec), _prec_name(t.precision()))
        if t.shape() != q.shape():
            raise ShapeMismatch("attention_backward", str(q.shape()), str(t.shape()))
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    ctx = q.ctx
    bh = b * h
    sc = Tensor.empty([bh, s, s], _P.FP32, ctx)
    p = Tensor.empty([bh, s, s], prec, ctx)
    dp = Tensor.empty([bh, s, s], _P.FP32, ctx)
    ds = Tensor.empty([bh, s, s], prec, ctx)
    dq = Tensor.empty([b, h, s, d], _P.FP32, ctx)
    dk = Tensor.empty([b, h, s, d], _P.FP32, ctx)
    dv = Tensor.empty([b, h, s, d], _P.FP32, ctx)
    lay = _layout_bhsd(s, d)
    check(ctx.lib.it_attention_backward(ctx.handle, int(prec), bh, s, d, float(scale), int(causal),
                                        C.byref(lay), None, None, _vp(grad_output), _vp(q), _vp(k), _vp(v),
                                        _vp(sc), _vp(p), _vp(dp), _vp(ds), _vp(dq), _vp(dk), _vp(dv)),
          "attention_backward")
    return dq, dk, dv


def flash_attention(q: Tensor, k: Tensor, v: Tensor, causal: bool) -> Tensor:
    """flash_attention (src/ops/flash_attention.rs:76-193, re-exported at src/ops/mod.rs:36 and
    src/lib.rs:32): softmax(Q.K^T / sqrt(head_dim), causal).V on [batch, heads, seq, head_dim] FP32
    tensors of one shape, head_dim <= 128, with the reference's assertions and messages; zeros at
    seq 0. head_dim 64 runs the fused kernels (the scores never leave the chip); other head sizes
    run the materialised contractions inside the same C entry point."""
    for name, t in (("Q", q), ("K", k), ("V", v)):
        if t.precision() is not _P.FP32:
            raise Panic(f"assertion `left == right` failed: {name} must be FP32")
    for name, t in (("Q", q), ("K", k), ("V", v)):
        if len(t.shape()) != 4:
            raise Panic(f"{name} must be 4D [batch, heads, seq, head_dim]")
    if q.shape() != k.shape():
        raise Panic("Q and K must have same shape")
    if q.shape() != v.shape():
        raise Panic("Q and V must have same shape")
    b, h, s, d = q.shape()
    if d > 128:
        raise Panic("head_dim must be <= 128")
    if b * h * s * d == 0:
        return Tensor.zeros([b, h, s, d], _P.FP32, q.ctx)
    out = Tensor.empty([b, h, s, d], _P.FP32, q.ctx)
    check(q.ctx.lib.it_flash_attention_forward(q.ctx.handle, _lib.IT_F32, b * h, s, s, d, 1.0 / math.sqrt(d),
                                               int(causal), None, None, None, _vp(q), _vp(k), _vp(v),
                                               _vp(out), None), "flash_attention")
    return out


def flash_attention_bshd(q: Tensor, k: Tensor, v: Tensor, causal: bool) -> Tensor:
    """ops::attention (src/ops/attention.rs:286-377) on [B,S,H,D] FP32 tensors through the fused entry
    point: for D = 64 the scores never leave the chip (online softmax over 64-key blocks); other
    D up to 128 run the materialised contractions. Same checks and panics as `attention`."""
    for t in (q, k, v):
        if t.precision() is not _P.FP32:
            raise Panic("assertion `left == right` failed: attention requires FP32")
    qs, ks, vs = q.shape(), k.shape(), v.shape()
    for name, sh in (("Q", qs), ("K", ks), ("V", vs)):
        if len(sh) != 4:
            raise Panic(f"{name} must be 4D [batch, seq, heads, dim]")
    b, sq, h, d = qs
    skv = ks[1]
    if ks[0] != b or vs[0] != b:
        raise Panic("Batch size mismatch")
    if ks[2] != h or vs[2] != h:
        raise Panic("Num heads mismatch")
    if ks[3] != d or vs[3] != d:
        raise Panic("Head dim mismatch")
    if vs[1] != skv:
        raise Panic("K and V seq_len must match")
    if b == 0 or sq == 0 or skv == 0:
        return Tensor.zeros([b, sq, h, d], _P.FP32, q.ctx)
    if causal and sq != skv:
        raise Panic("Causal attention requires Q and K to have same seq_len")
    out = Tensor.empty([b, sq, h, d], _P.FP32, q.ctx)
    lq, lkv = _layout_bshd(b, sq, h, d), _layout_bshd(b, skv, h, d)
    check(q.ctx.lib.it_flash_attention_forward(q.ctx.handle, _lib.IT_F32, b * h, sq, skv, d,
                                               1.0 / math.sqrt(d), int(causal), C.byref(lq),
                                               C.byref(lkv), C.byref(lq), _vp(q), _vp(k), _vp(v),
                                               _vp(out), None), "attention")
    return out


def flash_attention_forward_bhsd(q: Tensor, k: Tensor, v: Tensor, causal: bool = True,
                                 scale: Optional[float] = None,
                                 out_precision: Precision = _P.FP32) -> Tuple[Tensor, Tensor]:
    """Fused forward on [B,H,S,D] (D = 64, FP32 or BF16). Returns (O, lse f32 [B*H, S]); O is FP32,
    or BF16 with out_precision=BF16 (BF16 operands only)."""
    b, h, sq, d = q.shape()
    skv = k.shape()[2]
    prec = q.precision()
    for t in (k, v):
        if t.precision() is not prec:
            raise PrecisionMismatch("flash_attention", _prec_name(prec), _prec_name(t.precision()))
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    o = Tensor.empty([b, h, sq, d], out_precision, q.ctx)
    lse = Tensor.empty([b * h, sq], _P.FP32, q.ctx)
    lq, lkv = _layout_bhsd(sq, d), _layout_bhsd(skv, d)
    check(q.ctx.lib.it_flash_attention_forward_ex(q.ctx.handle, int(prec), int(out_precision), b * h, sq, skv, d,
                                                  float(scale), int(causal), C.byref(lq), C.byref(lkv),
                                                  C.byref(lq), _vp(q), _vp(k), _vp(v), _vp(o), _vp(lse)),
          "flash_attention")
    return o, lse


def flash_attention_backward(grad_output: Tensor, q: Tensor, k: Tensor, v: Tensor, causal: bool = True,
                             scale: Optional[float] = None, o: Optional[Tensor] = None,
                             lse: Optional[Tensor] = None,
                             out_precision: Precision = _P.FP32) -> Tuple[Tensor, Tensor, Tensor]:
    """attention_backward_recompute (src/train/helpers.rs:120-193) fused, on [B,H,S,D] (D = 64 fused;
    other D up to 128 recompute the materialised contractions). With `o` and `lse` from
    flash_attention_forward_bhsd (same out_precision) the forward is not recomputed. Returns
    (dQ, dK, dV), FP32 or, with out_precision=BF16 (BF16 operands, D = 64), BF16; deterministic (no
    atomics)."""
    b, h, s, d = q.shape()
    prec = q.precision()
    for t in (grad_output, k, v):
        if t.precision() is not prec:
            raise PrecisionMismatch("attention_backward", _prec_name(prec), _prec_name(t.precision()))
        if t.shape() != q.shape():
            raise ShapeMismatch("attention_backward", str(q.shape()), str(t.shape()))
    if (o is None) != (lse is None):
        raise InvalidValue("flash_attention_backward", "pass both o and lse, or neither")
    scale = 1.0 / math.sqrt(d) if scale is None else scale
    ctx = q.ctx
    dq = Tensor.empty([b, h, s, d], out_precision, ctx)
    dk = Tensor.empty([b, h, s, d], out_precision, ctx)
    dv = Tensor.empty([b, h, s, d], out_precision, ctx)
    lay = _layout_bhsd(s, d)
    check(ctx.lib.it_flash_attention_backward_ex(ctx.handle, int(prec), int(out_precision), b * h, s, d,
                                                 float(scale), int(causal), C.byref(lay), None, None,
                                                 _vp(grad_output), _vp(q), _vp(k), _vp(v),
                                                 _vp(o) if o is not None else None,
                                                 _vp(lse) if lse is not None else None,
                                                 _vp(dq), _vp(dk), _vp(dv)), "attention_backward")
    return dq, dk, dv


def transpose_3d_gpu(t: Tensor, batch: int, m: int, n: int) -> Tensor:
    """src/ops/attention.rs:395-449 (re-exported at src/ops/mod.rs:21): [batch, m, n] -> [batch, n, m],
    FP32, into a new tensor; panics unless t holds batch*m*n elements. The reference reads any
    tensor's buffer as f32; this mirror panics on a BF16 tensor instead of misreading it."""
    if t.numel() != batch * m * n:
        raise Panic("assertion `left == right` failed: Tensor size mismatch")
    if t.precision() is not _P.FP32:
        raise Panic("transpose_3d_gpu requires an FP32 tensor")
    out = Tensor.empty([batch, n, m], _P.FP32, t.ctx)
    check(t.ctx.lib.it_transpose_3d(t.ctx.handle, _vp(t), _vp(out), batch, m, n), "transpose_3d_gpu")
    return out


def causal_mask_3d_gpu(t: Tensor, batch: int, seq_len: int) -> Tensor:
    """src/ops/attention.rs:455-517 (re-exported at src/ops/mod.rs:21): [batch, seq, seq] scores with
    every column > row set to -inf, into a new FP32 tensor; panics unless t holds batch*seq*seq
    elements (a BF16 tensor panics too, where the reference would misread it as f32)."""
    if t.numel() != batch * seq_len * seq_len:
        raise Panic("assertion `left == right` failed: Tensor size mismatch")
    if t.precision() is not _P.FP32:
        raise Panic("causal_mask_3d_gpu requires an FP32 tensor")
    out = Tensor.empty([batch, seq_len, seq_len], _P.FP32, t.ctx)
    check(t.ctx.lib.it_causal_mask_3d(t.ctx.handle, _vp(t), _vp(out), batch, seq_len), "causal_mask_3d_gpu")
    return out


def softmax_rows(s: Tensor, causal: bool = False, out_precision: Precision = _P.FP32) -> Tensor:
    """Row softmax of an FP32 [.., rows, cols] tensor (src/shaders/softmax.metal), causal-aware."""
    shape = s.shape()
    rows, cols = shape[-2], shape[-1]
    batch = max(1, math.prod(shape[:-2]))
    out = Tensor.empty(shape, out_precision, s.ctx)
    check(s.ctx.lib.it_softmax_rows(s.ctx.handle, _vp(s), _vp(out), int(out_precision), batch, rows,
                                    cols, int(causal), 0), "softmax")
    return out


def softmax_backward(grad_output: Tensor, output: Tensor, causal: bool = False) -> Tensor:
    """src/ops/backward/softmax.rs / src/shaders/backward/softmax.metal:22-45."""
    shape = output.shape()
    rows, cols = shape[-2], shape[-1]
    batch = max(1, math.prod(shape[:-2]))
    out = Tensor.empty(shape, _P.FP32, output.ctx)
    check(output.ctx.lib.it_softmax_backward(output.ctx.handle, _vp(grad_output), _vp(output),
                                             int(output.precision()), _vp(out), _lib.IT_F32, batch,
                                             rows, cols, int(causal)), "softmax_backward")
    return out
