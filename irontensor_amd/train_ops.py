"""The reference's training-step ops around the contractions, on the MI355X C ABI.

Same names, argument meaning and error behaviour as IronTensor's Rust functions (each docstring
cites the function it mirrors); every op launches hand-written HIP through libirontensor_hip.so
(kernels_train.hip) and returns a new tensor as the reference does. There is no CPU fallback.
"""
from __future__ import annotations

import ctypes as C
from dataclasses import dataclass
from typing import List, Optional, Sequence, Tuple

import numpy as np

from .errors import Panic, PrecisionMismatch, check
from .tensor import Precision, Tensor

_P = Precision


def _vp(t: Optional[Tensor]):
    return C.c_void_p(t.ptr) if t is not None else C.c_void_p(0)


def _ids(indices, bound: int, what: str) -> Tuple[np.ndarray, Optional[Tensor]]:
    """Host index validation as the reference asserts it (src/ops/embedding.rs:41-49), then upload
    as uint32 (None when empty)."""
    ids = np.ascontiguousarray(np.asarray(indices, dtype=np.int64).ravel())
    bad = np.nonzero((ids < 0) | (ids >= bound))[0]
    if bad.size:
        i = int(bad[0])
        raise Panic(f"Index {int(ids[i])} at position {i} is out of bounds for {what} {bound}")
    return ids, (_upload_u32(ids) if ids.size else None)


def _upload_u32(ids: np.ndarray) -> Tensor:
    """uint32 ids in a device buffer (a [n] FP32-sized tensor holding the raw 32-bit words)."""
    return Tensor.from_f32_slice(ids.astype(np.uint32).view(np.float32), [ids.size])


def upload_ids(indices, bound: int, what: str = "vocab_size") -> Tensor:
    """Validated device copy of token ids or targets (uint32 words)."""
    return _ids(indices, bound, what)[1]


def _need_f32(t: Tensor, op: str, what: str = "input") -> None:
    if t.precision() is not _P.FP32:
        raise PrecisionMismatch(op, "FP32", t.precision().name)


def rmsnorm(input: Tensor, gamma: Tensor, eps: float, *, residual: Optional[Tensor] = None,
            sum_out: Optional[Tensor] = None, out_precision: Precision = _P.FP32) -> Tensor:
    """rmsnorm (src/ops/norm.rs:31): y = x / sqrt(mean(x^2) + eps) * gamma over the last dimension.

    With `residual`, x = input + residual first (the residual add of src/train/forward.rs:155,190,
    fused); `sum_out` receives that sum."""
    _need_f32(input, "rmsnorm")
    _need_f32(gamma, "rmsnorm", "gamma")
    dim = input.shape()[-1]
    if gamma.numel() != dim:
        raise Panic(f"gamma has {gamma.numel()} elements, expected {dim}")
    if residual is not None and residual.shape() != input.shape():
        raise Panic("residual shape differs from input")
    rows = input.numel() // max(dim, 1)
    y = Tensor.empty(input.shape(), out_precision, input.ctx)
    check(input.ctx.lib.it_rmsnorm_forward(input.ctx.handle, int(out_precision), rows, dim, float(eps),
                                           _vp(input), _vp(residual), _vp(gamma), _vp(sum_out), _vp(y)),
          "rmsnorm")
    return y


def rmsnorm_backward(grad_output: Tensor, input: Tensor, gamma: Tensor, eps: float, *,
                     residual_grad: Optional[Tensor] = None) -> Tuple[Tensor, Tensor]:
    """rmsnorm_backward (src/ops/backward/norm.rs:20) -> (grad_input, grad_gamma).

    With `residual_grad`, grad_input = residual_grad + the norm's input gradient (add_tensors at
    src/train/backward.rs:73,158, fused)."""
    for t in (grad_output, input, gamma):
        _need_f32(t, "rmsnorm_backward")
    if grad_output.shape() != input.shape():
        raise Panic("grad_output shape differs from input")
    dim = input.shape()[-1]
    rows = input.numel() // max(dim, 1)
    dx = Tensor.empty(input.shape(), _P.FP32, input.ctx)
    dg = Tensor.empty([dim], _P.FP32, input.ctx)
    check(input.ctx.lib.it_rmsnorm_backward(input.ctx.handle, rows, dim, float(eps), _vp(grad_output), _vp(input),
                                            _vp(gamma), _vp(residual_grad), _vp(dx), _vp(dg)), "rmsnorm_backward")
    return dx, dg


def fused_rmsnorm_linear(input: Tensor, gamma: Tensor, weight: Tensor, eps: float) -> Tensor:
    """fused_rmsnorm_linear (src/ops/fused_rmsnorm_linear.rs:73-205): rmsnorm(input, gamma, eps) @ weight^T
    without writing the normalized input. input [rows, hidden], weight [out_features, hidden], FP32."""
    for t in (input, gamma, weight):
        _need_f32(t, "fused_rmsnorm_linear")
    if len(input.shape()) != 2:
        raise Panic("Input must be 2D [batch_seq, hidden_dim]")
    if len(weight.shape()) != 2:
        raise Panic("Weight must be 2D [out_features, hidden_dim]")
    rows, hidden = input.shape()
    out_features, wh = weight.shape()
    if wh != hidden:
        raise Panic(f"Hidden dimensions must match: input has {hidden}, weight has {wh}")
    if gamma.shape() != [hidden]:
        raise Panic("Gamma must have shape [hidden_dim]")
    out = Tensor.empty([rows, out_features], _P.FP32, input.ctx)
    check(input.ctx.lib.it_fused_rmsnorm_linear(input.ctx.handle, rows, hidden, out_features, float(eps), _vp(input),
                                                _vp(gamma), _vp(weight), _vp(out)), "fused_rmsnorm_linear")
    return out


def _i32(targets) -> Tuple[np.ndarray, Optional[Tensor]]:
    t = np.ascontiguousarray(np.asarray(targets, dtype=np.int32).ravel())
    return t, (Tensor.from_f32_slice(t.view(np.float32), [t.size]) if t.size else None)


def fused_linear_cross_entropy(hidden: Tensor, weight: Tensor, targets, *, chunk_bytes: int = 0,
                               forward_only: bool = False):
    """fused_linear_cross_entropy (src/ops/fused_linear_cross_entropy.rs:79-242) -> (mean loss,
    grad_hidden, grad_weight); with forward_only, fused_linear_cross_entropy_forward_only (:246-374)
    -> (mean loss, grad_hidden). targets are i32; values outside [0, vocab) (-100) are ignored. The
    [rows, vocab] logits are never materialised (chunks of at most chunk_bytes, default 256 MiB).
    grad_weight is unscaled, as the reference's kernel leaves it."""
    _need_f32(hidden, "fused_linear_cross_entropy")
    _need_f32(weight, "fused_linear_cross_entropy")
    if len(hidden.shape()) != 2:
        raise Panic("hidden must be 2D [batch*seq, hidden_dim]")
    if len(weight.shape()) != 2:
        raise Panic("weight must be 2D [vocab_size, hidden_dim]")
    rows, hd = hidden.shape()
    vocab = weight.shape()[0]
    if weight.shape()[1] != hd:
        raise Panic("weight hidden_dim must match hidden")
    t_host, t = _i32(targets)
    if t_host.size != rows:
        raise Panic("targets length must match batch*seq")
    if hd > 256:
        raise Panic("hidden_dim must be <= 256 for this kernel")
    ctx = hidden.ctx
    gh = Tensor.zeros([rows, hd], _P.FP32, ctx)
    gw = None if forward_only else Tensor.zeros([vocab, hd], _P.FP32, ctx)
    mean = Tensor.zeros([1], _P.FP32, ctx)
    check(ctx.lib.it_fused_linear_cross_entropy(ctx.handle, rows, hd, vocab, _vp(hidden), _vp(weight), _vp(t), None,
                                                _vp(mean), _vp(gh), _vp(gw), int(chunk_bytes)),
          "fused_linear_cross_entropy")
    loss = float(mean.as_f32_slice()[0])
    return (loss, gh) if forward_only else (loss, gh, gw)


def _rope(x: Tensor, base: float, position_offset: int, backward: bool, name: str) -> Tensor:
    shape = x.shape()
    if len(shape) != 4:
        raise Panic(f"{name} expects [batch, seq, heads, head_dim], got {shape}")
    b, s, h, d = shape
    out = Tensor.empty(shape, x.precision(), x.ctx)
    check(x.ctx.lib.it_rope(x.ctx.handle, int(x.precision()), int(x.precision()), b, s, h, d, float(base),
                            int(position_offset), int(backward), _vp(x), h * d, _vp(out), h * d, 0), name)
    return out


def rope(input: Tensor, base: float, position_offset: int) -> Tensor:
    """rope (src/ops/rope.rs:22) over [batch, seq, heads, head_dim]."""
    return _rope(input, base, position_offset, False, "rope")


def rope_backward(grad_output: Tensor, base: float, position_offset: int) -> Tensor:
    """rope_backward (src/ops/backward/rope.rs:16): the transposed rotation."""
    return _rope(grad_output, base, position_offset, True, "rope_backward")


def embedding(weights: Tensor, indices) -> Tensor:
    """embedding (src/ops/embedding.rs:21): rows of weights [vocab, dim] gathered by index (FP32 out)."""
    shape = weights.shape()
    if len(shape) != 2:
        raise Panic("Weights must be 2D [vocab_size, embed_dim]")
    vocab, dim = shape
    ids_host, ids = _ids(indices, vocab, "vocab_size")
    out = Tensor.empty([ids_host.size, dim], _P.FP32, weights.ctx)
    check(weights.ctx.lib.it_embedding_forward(weights.ctx.handle, int(weights.precision()), int(_P.FP32),
                                               ids_host.size, dim, vocab, _vp(weights), _vp(ids), _vp(out)),
          "embedding")
    return out


def embedding_backward(grad_output: Tensor, indices, vocab_size: int) -> Tensor:
    """embedding_backward (src/ops/backward/embedding.rs:21): scatter-add into [vocab_size, dim]."""
    _need_f32(grad_output, "embedding_backward")
    shape = grad_output.shape()
    if len(shape) != 2:
        raise Panic("grad_output must be 2D")
    n, dim = shape
    ids_host, ids = _ids(indices, vocab_size, "vocab_size")
    if ids_host.size != n:
        raise Panic(f"assertion `left == right` failed\n  left: {ids_host.size}\n right: {n}")
    dw = Tensor.empty([vocab_size, dim], _P.FP32, grad_output.ctx)
    check(grad_output.ctx.lib.it_embedding_backward(grad_output.ctx.handle, n, dim, vocab_size, _vp(grad_output),
                                                    _vp(ids), _vp(dw)),
          "embedding_backward")
    return dw


def cross_entropy_fused(logits: Tensor, targets) -> Tuple[float, Tensor, Tensor]:
    """cross_entropy_fused (src/ops/backward/loss.rs:248) -> (mean loss, losses [rows], grad [rows, vocab])."""
    _need_f32(logits, "cross_entropy_fused")
    shape = logits.shape()
    if len(shape) != 2:
        raise Panic("logits must be 2D")
    rows, vocab = shape
    t_host, t = _ids(targets, vocab, "vocab_size")
    if t_host.size != rows:
        raise Panic(f"assertion `left == right` failed\n  left: {t_host.size}\n right: {rows}")
    losses = Tensor.zeros([rows], _P.FP32, logits.ctx)
    grad = Tensor.zeros(shape, _P.FP32, logits.ctx)
    if rows == 0:
        return 0.0, losses, grad
    mean = Tensor.empty([1], _P.FP32, logits.ctx)
    check(logits.ctx.lib.it_cross_entropy_fused(logits.ctx.handle, int(_P.FP32), rows, vocab, _vp(logits), _vp(t),
                                                _vp(losses), _vp(grad), _vp(mean)), "cross_entropy_fused")
    return float(mean.as_f32_slice()[0]), losses, grad


def cross_entropy_stats(logits: Tensor, targets) -> Tuple[float, Tensor, Tensor]:
    """The loss half of cross_entropy_fused (src/ops/backward/loss.rs:248) -> (mean loss, losses [rows],
    stats [rows, 2] = {max, 1 / sum exp(x - max)}); a GEMM with the IT_EPI_XENT_A operand rebuilds the
    gradient from the stats."""
    _need_f32(logits, "cross_entropy_stats")
    shape = logits.shape()
    if len(shape) != 2:
        raise Panic("logits must be 2D")
    rows, vocab = shape
    t_host, t = _ids(targets, vocab, "vocab_size")
    if t_host.size != rows:
        raise Panic(f"assertion `left == right` failed\n  left: {t_host.size}\n right: {rows}")
    losses = Tensor.zeros([rows], _P.FP32, logits.ctx)
    stats = Tensor.zeros([rows, 2], _P.FP32, logits.ctx)
    if rows == 0:
        return 0.0, losses, stats
    mean = Tensor.empty([1], _P.FP32, logits.ctx)
    check(logits.ctx.lib.it_cross_entropy_stats(logits.ctx.handle, rows, vocab, _vp(logits), _vp(t), _vp(losses),
                                                _vp(stats), _vp(mean)), "cross_entropy_stats")
    return float(mean.as_f32_slice()[0]), losses, stats


def swiglu_backward(grad_output: Tensor, gate: Tensor, up: Tensor) -> Tuple[Tensor, Tensor]:
    """swiglu_backward (src/ops/backward/elementwise.rs:149) -> (grad_gate, grad_up)."""
    _need_f32(grad_output, "swiglu_backward")
    if not (grad_output.shape() == gate.shape() == up.shape()):
        raise Panic("swiglu_backward: shapes differ")
    if gate.precision() is not up.precision():
        raise PrecisionMismatch("swiglu_backward", gate.precision().name, up.precision().name)
    cols = grad_output.shape()[-1] if grad_output.shape() else 1
    rows = grad_output.numel() // max(cols, 1)
    gg = Tensor.empty(gate.shape(), _P.FP32, gate.ctx)
    gu = Tensor.empty(gate.shape(), _P.FP32, gate.ctx)
    check(gate.ctx.lib.it_swiglu_backward(gate.ctx.handle, int(gate.precision()), int(_P.FP32), rows, cols,
                                          _vp(grad_output), cols, _vp(gate), _vp(up), cols, _vp(gg), _vp(gu), cols),
          "swiglu_backward")
    return gg, gu


def _ptr_table(tensors: Sequence[Tensor]):
    ptrs = (C.c_void_p * max(len(tensors), 1))(*[t.ptr for t in tensors])
    sizes = (C.c_int64 * max(len(tensors), 1))(*[t.numel() for t in tensors])
    return ptrs, sizes


def grad_norm_clip(tensors: Sequence[Tensor], max_norm: float, out: Tensor) -> None:
    """Device-side total L2 norm and clip factor into out[2] = {norm, scale} (no host sync)."""
    for t in tensors:
        _need_f32(t, "total_l2_norm_gpu")
    ctx = out.ctx
    ptrs, sizes = _ptr_table(tensors)
    check(ctx.lib.it_grad_norm_clip(ctx.handle, len(tensors), ptrs, sizes, float(max_norm), _vp(out)),
          "total_l2_norm_gpu")


def total_l2_norm_gpu(tensors: Sequence[Tensor]) -> float:
    """total_l2_norm_gpu (src/ops/reduction.rs:94): sqrt of the summed squares of all tensors."""
    if not tensors:
        return 0.0
    out = Tensor.empty([2], _P.FP32, tensors[0].ctx)
    grad_norm_clip(tensors, float("inf"), out)
    return float(out.as_f32_slice()[0])


@dataclass
class LionConfig:
    """LionConfig (src/optim/lion/config.rs:91-99 defaults); the benchmark's trainer uses lr 3e-4,
    beta1 0.9, beta2 0.99, weight_decay 0.1 (src/bin/benchmark.rs:124-129)."""
    lr: float = 1e-4
    beta1: float = 0.9
    beta2: float = 0.99
    weight_decay: float = 0.0


class ParamState:
    """Lion's per-parameter momentum (src/optim/lion/optimizer.rs: ParamState), zero-initialised."""

    def __init__(self, weights: Tensor):
        self.momentum = Tensor.zeros(weights.shape(), _P.FP32, weights.ctx)


class Lion:
    """Lion (src/optim/lion/optimizer.rs:32-106). `step` updates weights and momentum in place."""

    def __init__(self, config: LionConfig):
        self.config = config

    @staticmethod
    def with_lr(lr: float) -> "Lion":
        return Lion(LionConfig(lr=lr))

    def lr(self) -> float:
        return self.config.lr

    def set_lr(self, lr: float) -> None:
        self.config.lr = lr

    def step(self, weights: Tensor, gradients: Tensor, state: ParamState,
             grad_scale: Optional[Tensor] = None) -> None:
        self.step_many([weights], [gradients], [state], grad_scale)

    def step_many(self, weights: List[Tensor], gradients: List[Tensor], states: List[ParamState],
                  grad_scale: Optional[Tensor] = None, lr_dev: Optional[Tensor] = None) -> None:
        """One launch per 24 tensors; grad_scale (device [>=1] f32, e.g. the clip factor) multiplies
        every gradient first; lr_dev (device f32) overrides the configured learning rate."""
        if not (len(weights) == len(gradients) == len(states)):
            raise Panic("weights, gradients and states differ in length")
        for w, g in zip(weights, gradients):
            _need_f32(w, "lion")
            _need_f32(g, "lion")
            if w.numel() != g.numel():
                raise Panic(f"weights ({w.numel()}) and gradients ({g.numel()}) differ in size")
        if not weights:
            return
        ctx = weights[0].ctx
        wp, sizes = _ptr_table(weights)
        mp, _ = _ptr_table([s.momentum for s in states])
        gp, _ = _ptr_table(gradients)
        c = self.config
        check(ctx.lib.it_lion_step(ctx.handle, len(weights), wp, mp, gp, sizes, float(c.lr), float(c.beta1),
                                   float(c.beta2), float(c.weight_decay),
                                   C.c_void_p(grad_scale.ptr) if grad_scale is not None else C.c_void_p(0),
                                   C.c_void_p(lr_dev.ptr) if lr_dev is not None else C.c_void_p(0)), "lion")
