"""The contractions of one Llama-style training step at a model's real shapes, in step order on one
stream: the GEMM-set driver for the TINY and medium configurations.

Follows the reference trainer's call order (src/train/trainer/train_step.rs:39-236,
src/train/forward.rs:79-212, src/train/backward.rs:21-177) for every contraction it makes:

  forward, per layer:  QKV = X.Wqkv^T (one NT GEMM; the reference issues three, forward.rs:101-103)
                       attention contractions S = scale.Q.K^T (causal), P = softmax(S), O = P.V,
                       read in place from the QKV buffer's [B,S,H,D] layout (no transposes);
                       fused into one kernel for head_dim 64 (S and P stay on chip)
                       Y = O.Wo^T                                         (forward.rs:146)
                       h = silu(X2.Wg^T) * (X2.Wu^T), fused dual-B GEMM   (forward.rs:166-172)
                       Z = h.Wd^T                                         (forward.rs:175)
  LM head:             logits = Hf.E^T                                    (trainer/mod.rs:229-235)
  backward, LM head:   dE = dlogits^T.Hf (TN), dHf = dlogits.E (NN)       (train_step.rs:206-210)
  backward, per layer: down, gate|up (one GEMM each for dX and dW over the concatenated Wg|Wu),
                       Wo, attention_backward_recompute (5 GEMMs + softmax and its backward;
                       fused into dK/dV and dQ kernels for head_dim 64), QKV (backward.rs:53-147)

The elementwise work between contractions (RMSNorm, RoPE, residual adds, SwiGLU backward, cross
entropy) is outside this path: each layer's normalised inputs and each upstream gradient are
seeded N(0,1) buffers standing where those ops would write, so every GEMM runs at its real shape
on realistic data. Weights are N(0, 0.02); all seeded inputs are drawn on the device
(synth.normal_tensor), the same stream as the host's synth.normal.
"""
from __future__ import annotations

import ctypes as C
import math
from dataclasses import dataclass
from typing import List, Optional, Tuple

import numpy as np

from . import _lib, synth
from .errors import check
from .tensor import Context, Precision, Tensor


@dataclass(frozen=True)
class ModelShape:
    name: str
    layers: int
    hidden: int
    heads: int
    head_dim: int
    ffn: int
    vocab: int
    batch: int
    seq: int

    @property
    def tokens(self) -> int:
        return self.batch * self.seq


# BASELINE configs[1] and configs[3]
TINY = ModelShape("tiny", 4, 256, 4, 64, 688, 16384, 16, 256)
MEDIUM = ModelShape("medium", 12, 1024, 16, 64, 2816, 32768, 8, 1024)


class _Launch:
    """One recorded contraction for reporting: name and dense-equivalent FLOPs."""

    __slots__ = ("name", "flops")

    def __init__(self, name: str, flops: float):
        self.name, self.flops = name, flops


class GemmStep:
    """Owns every buffer of the step and enqueues its contractions (eagerly or into a HIP graph)."""

    def __init__(self, shape: ModelShape, precision: Precision = Precision.FP32,
                 ctx: Optional[Context] = None, seed: int = 1234, fused_attention: Optional[bool] = None,
                 ffn_bias: bool = False, overlap_weight_grads: bool = False):
        if shape.heads * shape.head_dim != shape.hidden:
            raise ValueError("heads * head_dim must equal hidden")
        self.s = shape
        self.prec = Precision(precision)
        self.ctx = ctx or Context.global_()
        self.lib = self.ctx.lib
        self.graph = None
        s, P = shape, self.prec
        T, H, F, V, L = s.tokens, s.hidden, s.ffn, s.vocab, s.layers
        bh = s.batch * s.heads
        self._seed = seed
        # Seeded inputs are generated on the device (synth.normal_tensor: the stream of synth.normal);
        # seed_of maps each one's device address to (seed, std), so a check can regenerate any
        # element on the host (synth.normal_at).
        self.seed_of: dict = {}
        # A layer's four weight gradients are issued together, once its last upstream gradient
        # (dQKV) is ready, and go to the library as one group (it_gemm_group): one launch that
        # fills the GPU, so they run on the main stream by default. With overlap_weight_grads they
        # run on the context's side stream instead, beside the data-gradient chain (one fork per
        # layer: each fork idles the GPU for microseconds inside the graph; dw_fork = "gemm" forks
        # per GEMM).
        self.overlap = overlap_weight_grads
        self.dw_fork = "layer"
        self.group_weight_grads = True
        self._dw_queue = None
        self._first_group = None

        def w(shape_, std=0.02):
            return self._tensor(shape_, std)

        def act(shape_):
            return self._tensor(shape_, 1.0)

        def empty(shape_, prec=P):
            return Tensor.empty(shape_, prec, self.ctx)

        # Weights (layer-major lists), stored as the reference stores them: [out, in].
        self.Wqkv = [w([3 * H, H]) for _ in range(L)]
        self.Wo = [w([H, H]) for _ in range(L)]
        self.Wgu = [w([2 * F, H]) for _ in range(L)]   # gate rows then up rows
        self.Wd = [w([H, F]) for _ in range(L)]
        # Optional gate|up biases (FP32 [2F]) applied in the fused SwiGLU epilogue
        self.bgu = [Tensor.from_f32_slice(synth.normal(self._seed + 7 + l, (2 * F,), std=0.02), [2 * F],
                                          self.ctx) for l in range(L)] if ffn_bias else None
        self.E = w([V, H])                             # untied LM head
        # Forward caches
        self.X = [act([T, H]) for _ in range(L)]       # attention-norm output
        self.X2 = [act([T, H]) for _ in range(L)]      # ffn-norm output
        self.QKV = [empty([T, 3 * H]) for _ in range(L)]
        # The attention output feeds the output projection and dQ|dK|dV the QKV projection's
        # backward (src/train/forward.rs:138-146, src/train/backward.rs:100-147). In BF16 the fused
        # kernels write them as BF16 (it_flash_attention_*_ex); the materialised form writes FP32,
        # so with it a BF16 step's two projections read seeded BF16 stand-ins instead.
        self.fused = (s.head_dim == 64) if fused_attention is None else bool(fused_attention)
        self.attn_out = P if (self.fused or P is Precision.FP32) else Precision.FP32
        self.O = [empty([T, H], self.attn_out) for _ in range(L)]
        self.Oin = self.O if self.attn_out is P else [act([T, H]) for _ in range(L)]
        self.Y = [empty([T, H]) for _ in range(L)]
        self.G = [empty([T, F]) for _ in range(L)]
        self.U = [empty([T, F]) for _ in range(L)]
        self.Hh = [empty([T, F]) for _ in range(L)]
        self.Z = [empty([T, H]) for _ in range(L)]
        self.Hf = act([T, H])
        self.logits = empty([T, V])
        # Backward: upstream gradients (seeded) and results
        self.dlogits = act([T, V])
        self.dZ = act([T, H])
        self.dGU = act([T, 2 * F])
        self.dY = act([T, H])
        self.dO = act([T, H])
        self.dE = empty([V, H], Precision.FP32)
        self.dHf = empty([T, H], Precision.FP32)
        self.dHh = empty([T, F], Precision.FP32)
        self.dX2 = empty([T, H], Precision.FP32)
        self.dOp = empty([T, H], Precision.FP32)
        # One dQKV per layer: a layer's qkv.dW (side stream) may still read it while the next layer's
        # attention backward (main stream) writes its own.
        self.dQKV_layers = [empty([T, 3 * H], self.attn_out) for _ in range(L)]
        self.dQKV = self.dQKV_layers[0]
        self.dX = empty([T, H], Precision.FP32)
        self.dWd = [empty([H, F], Precision.FP32) for _ in range(L)]
        self.dWgu = [empty([2 * F, H], Precision.FP32) for _ in range(L)]
        self.dWo = [empty([H, H], Precision.FP32) for _ in range(L)]
        self.dWqkv = [empty([3 * H, H], Precision.FP32) for _ in range(L)]
        # Attention: the fused kernels keep each layer's row log-sum-exp for the backward; the
        # materialised form needs [BH, S, S] workspaces, shared by all layers.
        if self.fused:
            self.lse = [empty([bh, s.seq], Precision.FP32) for _ in range(L)]
        else:
            self.Sc = empty([bh, s.seq, s.seq], Precision.FP32)
            self.Pw = empty([bh, s.seq, s.seq])
            self.dP = empty([bh, s.seq, s.seq], Precision.FP32)
            self.dS = empty([bh, s.seq, s.seq])
        self.launches: List[_Launch] = []
        self._calls: dict = {}
        self._record = True

    # ---------------------------------------------------------------- helpers
    def _tensor(self, shape_, std) -> Tensor:
        self._seed += 1
        t = synth.normal_tensor(self._seed, shape_, std=std, precision=self.prec, ctx=self.ctx)
        self.seed_of[t.ptr] = (self._seed, std)
        return t

    def _call(self, A: Tensor, B: Tensor, Cout: Tensor, ta: bool, tb: bool, M, N, K, alpha=1.0,
              epi: Optional[_lib.Epilogue] = None, a_off=0, lda=None) -> _lib.GemmCall:
        """it_gemm's arguments for one GEMM of the step (batch 1, beta 0)."""
        lda = lda if lda is not None else (A.shape()[-1])
        eb = self.prec.byte_size()
        return _lib.GemmCall(int(ta), int(tb), M, N, K, float(alpha), A.ptr + a_off * eb, lda, 0, B.ptr,
                             B.shape()[-1], 0, 0.0, Cout.ptr, Cout.shape()[-1], 0, 1,
                             C.pointer(epi) if epi is not None else None)

    def _gemm(self, name, A: Tensor, B: Tensor, Cout: Tensor, ta: bool, tb: bool, M, N, K,
              alpha=1.0, epi: Optional[_lib.Epilogue] = None, a_off=0, lda=None):
        c = self._call(A, B, Cout, ta, tb, M, N, K, alpha, epi, a_off, lda)
        st = self.lib.it_gemm(self.ctx.handle, int(self.prec), int(Cout.precision()), c.transA, c.transB, M, N, K,
                              c.alpha, c.A, c.lda, 0, c.B, c.ldb, 0, 0.0, c.C, c.ldc, 0, 1,
                              C.byref(epi) if epi is not None else None)
        check(st, name)
        self._note(name, A, B, Cout, ta, tb, M, N, K, alpha, epi, a_off, lda)

    def _note(self, name, A, B, Cout, ta, tb, M, N, K, alpha=1.0, epi=None, a_off=0, lda=None):
        """The step's bookkeeping of one GEMM: its FLOPs and the first call of each shape."""
        lda = lda if lda is not None else (A.shape()[-1])
        if self._record:
            mult = 2 if (epi is not None and epi.flags & _lib.IT_EPI_SWIGLU) else 1
            self.launches.append(_Launch(name, 2.0 * M * N * K * mult))
            key = (bool(ta), bool(tb), M, N, K)
            if key not in self._calls:
                self._calls[key] = (name, A, B, Cout, ta, tb, M, N, K, alpha, epi, a_off, lda)

    def _dw(self, *args, **kw):
        """A weight-gradient GEMM: queued for the layer's group when one is open (issued together
        at the end of the layer), else on the side stream when overlapping."""
        if self._dw_queue is not None:
            self._dw_queue.append((args, kw))
            return None
        if not self.overlap:
            return self._gemm(*args, **kw)
        check(self.lib.it_side_begin(self.ctx.handle), "side stream")
        try:
            self._gemm(*args, **kw)
        finally:
            check(self.lib.it_side_end(self.ctx.handle), "side stream")

    def _dw_flush(self):
        """The layer's queued weight gradients (on the side stream when overlapping), as one
        it_gemm_group call (one launch where the library can group them, else one GEMM after the
        other)."""
        q, self._dw_queue = self._dw_queue, None
        if not q:
            return
        if self.overlap:
            check(self.lib.it_side_begin(self.ctx.handle), "side stream")
        try:
            if self.group_weight_grads and len({a[3].precision() for a, _ in q}) == 1:
                self._issue_group(q)
                if self._record and self._first_group is None:
                    self._first_group = q
                for args, kw in q:
                    self._note(*args, **kw)
            else:
                for args, kw in q:
                    self._gemm(*args, **kw)
        finally:
            if self.overlap:
                check(self.lib.it_side_end(self.ctx.handle), "side stream")

    def _issue_group(self, q) -> None:
        calls = (_lib.GemmCall * len(q))(*[self._call(*a[1:], **kw) for a, kw in q])
        check(self.lib.it_gemm_group(self.ctx.handle, int(self.prec), int(q[0][0][3].precision()), len(q), calls),
              "weight gradients")

    def reissue_group(self) -> List[str]:
        """Launches again the first layer's weight-gradient group as issued in the step (one
        it_gemm_group call, for profiling it in isolation); returns the names of its GEMMs.
        enqueue() must have run once with grouped weight gradients."""
        if self._first_group is None:
            raise RuntimeError("no weight-gradient group was issued")
        self._issue_group(self._first_group)
        return [a[0] for a, _ in self._first_group]

    def _layouts(self):
        s = self.s
        qkv = _lib.AttnLayout(s.heads, s.seq * 3 * s.hidden, s.head_dim, 3 * s.hidden)
        o = _lib.AttnLayout(s.heads, s.seq * s.hidden, s.head_dim, s.hidden)
        return qkv, o

    # ---------------------------------------------------------------- the step
    def forward_layer(self, l: int) -> None:
        s, P = self.s, self.prec
        T, H, F = s.tokens, s.hidden, s.ffn
        eb = P.byte_size()
        self._gemm("qkv", self.X[l], self.Wqkv[l], self.QKV[l], False, True, T, 3 * H, H)
        qkv, o = self._layouts()
        base = self.QKV[l].ptr
        q, k, v = (C.c_void_p(base + i * H * eb) for i in range(3))
        if self.fused:
            st = self.lib.it_flash_attention_forward_ex(
                self.ctx.handle, int(P), int(self.attn_out), s.batch * s.heads, s.seq, s.seq, s.head_dim,
                1.0 / math.sqrt(s.head_dim), 1, C.byref(qkv), C.byref(qkv), C.byref(o), q, k, v,
                C.c_void_p(self.O[l].ptr), C.c_void_p(self.lse[l].ptr))
        else:
            st = self.lib.it_attention_forward(
                self.ctx.handle, int(P), s.batch * s.heads, s.seq, s.seq, s.head_dim,
                1.0 / math.sqrt(s.head_dim), 1, C.byref(qkv), C.byref(qkv), C.byref(o), q, k, v,
                C.c_void_p(self.Sc.ptr), C.c_void_p(self.Pw.ptr), C.c_void_p(self.O[l].ptr))
        check(st, "attention")
        if self._record:
            attn = 2.0 * s.batch * s.heads * s.seq * s.seq * s.head_dim
            self.launches += [_Launch("attn.S", attn), _Launch("attn.O", attn)]
        self._gemm("wo", self.Oin[l], self.Wo[l], self.Y[l], False, True, T, H, H)
        epi = _lib.Epilogue(flags=_lib.IT_EPI_SWIGLU, B2=self.Wgu[l].ptr + F * H * eb,
                            gate_out=self.G[l].ptr, up_out=self.U[l].ptr)
        if self.bgu is not None:
            epi.flags |= _lib.IT_EPI_BIAS
            epi.bias = self.bgu[l].ptr
        self._gemm("gate_up_swiglu", self.X2[l], self.Wgu[l], self.Hh[l], False, True, T, F, H, epi=epi)
        self._gemm("down", self.Hh[l], self.Wd[l], self.Z[l], False, True, T, H, F)

    def backward_layer(self, l: int) -> None:
        s, P = self.s, self.prec
        T, H, F = s.tokens, s.hidden, s.ffn
        if (self.overlap and self.dw_fork == "layer") or self.group_weight_grads:
            self._dw_queue = []
        # down: dHh = dZ.Wd (NN), dWd = dZ^T.Hh (TN)
        self._dw("down.dW", self.dZ, self.Hh[l], self.dWd[l], True, False, H, F, T)
        self._gemm("down.dX", self.dZ, self.Wd[l], self.dHh, False, False, T, F, H)
        # gate|up: dX2 = [dG dU].[Wg;Wu] (NN, K = 2F), dWgu = [dG dU]^T.X2 (TN)
        self._dw("gate_up.dW", self.dGU, self.X2[l], self.dWgu[l], True, False, 2 * F, H, T)
        self._gemm("gate_up.dX", self.dGU, self.Wgu[l], self.dX2, False, False, T, H, 2 * F)
        # Wo: dO = dY.Wo (NN), dWo = dY^T.O (TN)
        self._dw("wo.dW", self.dY, self.Oin[l], self.dWo[l], True, False, H, H, T)
        self._gemm("wo.dX", self.dY, self.Wo[l], self.dOp, False, False, T, H, H)
        # attention_backward_recompute into the layer's dQKV buffer (same [B,S,3,H,D] layout as QKV)
        qkv, o = self._layouts()
        eb = P.byte_size()
        base = self.QKV[l].ptr
        dbase = self.dQKV_layers[l].ptr
        q, k, v = (C.c_void_p(base + i * H * eb) for i in range(3))
        dq, dk, dv = (C.c_void_p(dbase + i * H * self.attn_out.byte_size()) for i in range(3))
        if self.fused:
            st = self.lib.it_flash_attention_backward_ex(
                self.ctx.handle, int(P), int(self.attn_out), s.batch * s.heads, s.seq, s.head_dim,
                1.0 / math.sqrt(s.head_dim), 1, C.byref(qkv), C.byref(qkv), C.byref(o),
                C.c_void_p(self.dO.ptr), q, k, v, C.c_void_p(self.O[l].ptr),
                C.c_void_p(self.lse[l].ptr), dq, dk, dv)
        else:
            st = self.lib.it_attention_backward(
                self.ctx.handle, int(P), s.batch * s.heads, s.seq, s.head_dim,
                1.0 / math.sqrt(s.head_dim), 1, C.byref(qkv), C.byref(qkv), C.byref(o),
                C.c_void_p(self.dO.ptr), q, k, v, C.c_void_p(self.Sc.ptr), C.c_void_p(self.Pw.ptr),
                C.c_void_p(self.dP.ptr), C.c_void_p(self.dS.ptr), dq, dk, dv)
        check(st, "attention_backward")
        if self._record:
            attn = 2.0 * s.batch * s.heads * s.seq * s.seq * s.head_dim
            self.launches += [_Launch(n, attn) for n in ("attn.S", "attn.dV", "attn.dP", "attn.dQ", "attn.dK")]
        # QKV: dX = dQKV.Wqkv (NN), dWqkv = dQKV^T.X (TN), reading the attention backward's dQ|dK|dV
        # (the materialised form's FP32 gradient leaves a BF16 step a seeded BF16 stand-in).
        dqkv = self.dQKV_layers[l] if self.attn_out is P else self._dqkv_bf16()
        self._dw("qkv.dW", dqkv, self.X[l], self.dWqkv[l], True, False, 3 * H, H, T)
        self._dw_flush()
        self._gemm("qkv.dX", dqkv, self.Wqkv[l], self.dX, False, False, T, H, 3 * H)

    def _dqkv_bf16(self) -> Tensor:
        if not hasattr(self, "_dqkv16"):
            self._dqkv16 = self._tensor([self.s.tokens, 3 * self.s.hidden], 1.0)
        return self._dqkv16

    def enqueue(self) -> None:
        """Issues one full step on the context stream."""
        s = self.s
        self._dw_queue = None  # a step interrupted mid-layer leaves no queued weight gradients
        if self._record:
            self.launches = []
        for l in range(s.layers):
            self.forward_layer(l)
        self._gemm("lm_head", self.Hf, self.E, self.logits, False, True, s.tokens, s.vocab, s.hidden)
        self._dw("lm_head.dW", self.dlogits, self.Hf, self.dE, True, False, s.vocab, s.hidden, s.tokens)
        self._gemm("lm_head.dX", self.dlogits, self.E, self.dHf, False, False, s.tokens, s.hidden, s.vocab)
        for l in reversed(range(s.layers)):
            self.backward_layer(l)
        if self.overlap:
            check(self.lib.it_side_join(self.ctx.handle), "side stream")
        self._record = False

    def reissue(self, ta: bool, tb: bool, M: int, N: int, K: int) -> str:
        """Launches again the first GEMM of the step with this layout and shape (for profiling one
        kernel in isolation); returns its name. enqueue() must have run once."""
        name, A, B, Cout, ta_, tb_, M_, N_, K_, alpha, epi, a_off, lda = self._calls[(ta, tb, M, N, K)]
        rec, self._record = self._record, False
        try:
            self._gemm(name, A, B, Cout, ta_, tb_, M_, N_, K_, alpha=alpha, epi=epi, a_off=a_off, lda=lda)
        finally:
            self._record = rec
        return name

    def flops(self) -> float:
        return float(sum(x.flops for x in self.launches))

    def capture(self) -> None:
        """Captures one step into a HIP graph (run enqueue() once first so scratch is sized)."""
        check(self.lib.it_capture_begin(self.ctx.handle), "capture")
        try:
            self.enqueue()
        finally:
            g = C.c_void_p()
            st = self.lib.it_capture_end(self.ctx.handle, C.byref(g))
        check(st, "capture")
        self.graph = g

    def replay(self) -> None:
        check(self.lib.it_graph_launch(self.ctx.handle, self.graph), "graph launch")

    def close(self) -> None:
        if self.graph is not None:
            self.lib.it_graph_destroy(self.graph)
            self.graph = None
