"""One complete Llama-style training step on the GPU: embedding, transformer layers, final norm, LM
head, fused cross entropy, the backward pass, global-norm gradient clipping and Lion, in the
reference trainer's order (src/train/trainer/train_step.rs:39-460, src/train/forward.rs:79-212,
src/train/backward.rs:21-177), FP32.

Every op is a hand-written HIP kernel behind the C ABI: the contractions (it_gemm, the fused
attention kernels), and the row/elementwise ops of kernels_train.hip. The MI355X-specific choices:

  * residual adds are fused into the RMSNorm that follows them (forward) and the RMSNorm backward
    that precedes them (backward), so no standalone add kernel runs;
  * Q|K|V is one NT GEMM into a [T, 3H] buffer with RoPE applied to Q and K in its epilogue;
    attention reads heads from it by stride, and its backward writes dQ|dK|dV into one [T, 3H]
    buffer that RoPE's backward rotates in place and one NN GEMM consumes;
  * gate and up are one dual-B GEMM with the SwiGLU epilogue; the down projection's dX GEMM runs
    the SwiGLU backward in its epilogue, writing the [T, 2F] gate|up gradient read by one NN and
    one TN GEMM (dL/dh is never stored);
  * cross entropy writes the [T, V] logit gradient once and the two LM-head backward GEMMs read it;
    with xent_operand=True it writes only the loss and each row's {max, 1/sum}, and both GEMMs
    rebuild the gradient from the logits on their way into LDS (IT_EPI_XENT_A): 268 MB less at
    TINY, but slower (the rebuild runs once per output tile column: cross entropy 111 -> 43 us,
    the dX and dW GEMMs 298 -> 418 and 287 -> 342 us on MI355X), so it is off by default;
  * a layer's four weight-gradient GEMMs are issued together once their last input (the RoPE
    backward) is ready, as one it_gemm_group call (one launch with one split-K reduction where the
    library's model prices that below four separate plans). Every buffer they read is per layer,
    so the main stream never overwrites one before they have read it. They run on the main stream
    by default; overlap_weight_grads puts them on the side stream beside the data-gradient chain,
    forked once per layer (dw_fork="layer": each fork costs several microseconds of idle GPU
    inside the graph, so that beat one fork per GEMM, "gemm", 2.80 against 2.85 ms per TINY step
    before the grouping);
  * the gradient norm, the clip factor and the learning rate stay on the device (Lion reads them
    from memory), so a step has no host synchronisation and captures into one HIP graph.

Untied LM head (BASELINE's TINY configuration): the input embedding and the output projection are
separate [V, H] matrices. (The reference's trainer multiplies by the input embedding and, with
tie_weights off, drops that product's gradient, src/train/trainer/train_step.rs:83-87.)
"""
from __future__ import annotations

import ctypes as C
import math
from typing import List, Optional

import numpy as np

from . import _lib, synth
from .errors import check
from .step import ModelShape, TINY
from .tensor import Context, Precision, Tensor

_F32 = Precision.FP32


class TrainStep:
    """Owns parameters, optimizer state, activations and gradients; enqueues one full step."""

    def __init__(self, shape: ModelShape = TINY, ctx: Optional[Context] = None, seed: int = 1234,
                 lr: float = 3e-4, beta1: float = 0.9, beta2: float = 0.99, weight_decay: float = 0.1,
                 max_grad_norm: float = 1.0, eps: float = 1e-5, rope_base: float = 10000.0,
                 overlap_weight_grads: bool = False, fused_attention: Optional[bool] = None,
                 xent_operand: bool = False, dw_fork: str = "layer", group_weight_grads: bool = True):
        s = shape
        if s.heads * s.head_dim != s.hidden:
            raise ValueError("heads * head_dim must equal hidden")
        self.s = s
        self.ctx = ctx or Context.global_()
        self.lib = self.ctx.lib
        self.h = self.ctx.handle
        self.eps, self.rope_base = float(eps), float(rope_base)
        self.lr, self.beta1, self.beta2, self.wd = float(lr), float(beta1), float(beta2), float(weight_decay)
        self.max_grad_norm = float(max_grad_norm)
        self.overlap = overlap_weight_grads
        self.group_weight_grads = bool(group_weight_grads)
        self.fused = (s.head_dim == 64) if fused_attention is None else bool(fused_attention)
        self.xent_operand = bool(xent_operand)
        if dw_fork not in ("gemm", "layer"):
            raise ValueError("dw_fork is 'gemm' or 'layer'")
        self.dw_fork = dw_fork
        self._dw_queue = None
        self.graph = None
        self._seed = seed
        T, H, F, V, L = s.tokens, s.hidden, s.ffn, s.vocab, s.layers
        bh = s.batch * s.heads

        def w(shape_, std=0.02):
            self._seed += 1
            return Tensor.from_f32_slice(synth.normal(self._seed, shape_, std=std), shape_, self.ctx)

        def ones(n):
            return Tensor.from_f32_slice(np.ones(n, np.float32), [n], self.ctx)

        def empty(shape_):
            return Tensor.empty(shape_, _F32, self.ctx)

        # ---- parameters, stored as the reference stores them ([out, in] weights)
        self.emb = w([V, H])
        self.attn_norm = [ones(H) for _ in range(L)]
        self.ffn_norm = [ones(H) for _ in range(L)]
        self.Wqkv = [w([3 * H, H]) for _ in range(L)]
        self.Wo = [w([H, H]) for _ in range(L)]
        self.Wgu = [w([2 * F, H]) for _ in range(L)]   # gate rows, then up rows
        self.Wd = [w([H, F]) for _ in range(L)]
        self.final_norm = ones(H)
        self.E = w([V, H])
        self.params: List[Tensor] = [self.emb, self.final_norm, self.E]
        for l in range(L):
            self.params += [self.attn_norm[l], self.ffn_norm[l], self.Wqkv[l], self.Wo[l], self.Wgu[l], self.Wd[l]]
        self.momentum = [Tensor.zeros(p.shape(), _F32, self.ctx) for p in self.params]

        # ---- gradients (same order as params)
        self.d_emb, self.d_final_norm, self.dE = empty([V, H]), empty([H]), empty([V, H])
        self.d_attn_norm = [empty([H]) for _ in range(L)]
        self.d_ffn_norm = [empty([H]) for _ in range(L)]
        self.dWqkv = [empty([3 * H, H]) for _ in range(L)]
        self.dWo = [empty([H, H]) for _ in range(L)]
        self.dWgu = [empty([2 * F, H]) for _ in range(L)]
        self.dWd = [empty([H, F]) for _ in range(L)]
        self.grads: List[Tensor] = [self.d_emb, self.d_final_norm, self.dE]
        for l in range(L):
            self.grads += [self.d_attn_norm[l], self.d_ffn_norm[l], self.dWqkv[l], self.dWo[l], self.dWgu[l],
                           self.dWd[l]]

        # ---- batch (device uint32 ids and targets), device scalars
        self.ids = Tensor.empty([T], _F32, self.ctx)
        self.targets = Tensor.empty([T], _F32, self.ctx)
        self.loss = empty([1])
        self.losses = empty([T])
        self.norm_clip = empty([2])        # {global grad norm, clip factor}
        self.lr_dev = Tensor.from_f32_slice(np.array([self.lr], np.float32), [1], self.ctx)

        # ---- forward activations
        self.xin = [empty([T, H]) for _ in range(L + 1)]  # layer inputs; xin[L] = last layer's output
        self.xn = [empty([T, H]) for _ in range(L)]
        self.QKV = [empty([T, 3 * H]) for _ in range(L)]
        self.O = [empty([T, H]) for _ in range(L)]
        self.post = [empty([T, H]) for _ in range(L)]
        self.x2 = [empty([T, H]) for _ in range(L)]
        self.G = [empty([T, F]) for _ in range(L)]
        self.U = [empty([T, F]) for _ in range(L)]
        self.Hh = [empty([T, F]) for _ in range(L)]
        self.Y = empty([T, H])   # attention projection, consumed at once by the fused add+norm
        self.Z = empty([T, H])   # FFN output, likewise
        self.Hf = empty([T, H])
        self.logits = empty([T, V])
        if self.xent_operand:
            self.ce_stats = empty([T, 2])   # per token {max, 1 / sum exp(x - max)}
        else:
            self.dlogits = empty([T, V])
        if self.fused:
            self.lse = [empty([bh, s.seq]) for _ in range(L)]
        else:
            self.Sc, self.dP = empty([bh, s.seq, s.seq]), empty([bh, s.seq, s.seq])
            self.Pw, self.dS = empty([bh, s.seq, s.seq]), empty([bh, s.seq, s.seq])

        # ---- backward: per-layer buffers the side stream reads
        self.g_out = [empty([T, H]) for _ in range(L + 1)]  # gradient w.r.t. xin[l]; g_out[L] from the final norm
        self.gpost = [empty([T, H]) for _ in range(L)]
        self.dGU = [empty([T, 2 * F]) for _ in range(L)]
        self.dQKV = [empty([T, 3 * H]) for _ in range(L)]
        self.dX2 = empty([T, H])
        self.dOp = empty([T, H])
        self.dXn = empty([T, H])
        self.dHf = empty([T, H])
        self.set_batch(*self.synthetic_batch(seed))

    # ---------------------------------------------------------------- data
    def synthetic_batch(self, seed: int):
        """Uniform random tokens: per sequence, seq+1 consecutive tokens of a
        seeded stream give the inputs and the next-token targets."""
        s = self.s
        stream = synth.tokens(seed + 777, s.batch * (s.seq + 1), s.vocab).reshape(s.batch, s.seq + 1)
        return stream[:, :-1].ravel(), stream[:, 1:].ravel()

    def set_batch(self, ids, targets) -> None:
        ids = np.ascontiguousarray(np.asarray(ids, dtype=np.int64).ravel())
        targets = np.ascontiguousarray(np.asarray(targets, dtype=np.int64).ravel())
        T, V = self.s.tokens, self.s.vocab
        if ids.size != T or targets.size != T:
            raise ValueError(f"a batch holds {T} ids and {T} targets")
        if ids.min() < 0 or ids.max() >= V or targets.min() < 0 or targets.max() >= V:
            raise ValueError("token id out of range")
        self.ids_host, self.targets_host = ids.astype(np.uint32), targets.astype(np.uint32)
        for dev, host in ((self.ids, self.ids_host), (self.targets, self.targets_host)):
            check(self.lib.it_memcpy_h2d(self.h, C.c_void_p(dev.ptr), host.ctypes.data_as(C.c_void_p), host.nbytes),
                  "upload batch")

    def set_lr(self, lr: float) -> None:
        """Learning rate for the next step (a device value: graph replays pick it up)."""
        self.lr = float(lr)
        v = np.array([self.lr], np.float32)
        check(self.lib.it_memcpy_h2d(self.h, C.c_void_p(self.lr_dev.ptr), v.ctypes.data_as(C.c_void_p), 4), "lr")

    # ---------------------------------------------------------------- launch helpers
    @staticmethod
    def _call(A: Tensor, B: Tensor, Cout: Tensor, ta: bool, tb: bool, M, N, K,
              epi: Optional[_lib.Epilogue] = None) -> _lib.GemmCall:
        """it_gemm's arguments for one FP32 GEMM of the step (batch 1, alpha 1, beta 0)."""
        return _lib.GemmCall(int(ta), int(tb), M, N, K, 1.0, A.ptr, A.shape()[-1], 0, B.ptr, B.shape()[-1], 0,
                             0.0, Cout.ptr, Cout.shape()[-1], 0, 1, C.pointer(epi) if epi is not None else None)

    def _gemm(self, name, A: Tensor, B: Tensor, Cout: Tensor, ta: bool, tb: bool, M, N, K,
              epi: Optional[_lib.Epilogue] = None):
        st = self.lib.it_gemm(self.h, 0, 0, int(ta), int(tb), M, N, K, 1.0, C.c_void_p(A.ptr), A.shape()[-1], 0,
                              C.c_void_p(B.ptr), B.shape()[-1], 0, 0.0, C.c_void_p(Cout.ptr), Cout.shape()[-1], 0, 1,
                              C.byref(epi) if epi is not None else None)
        check(st, name)

    def _dw(self, *args, **kw):
        """A weight-gradient GEMM: queued and issued with the rest of its layer's when a queue is
        open (group_weight_grads, or dw_fork="layer" on the side stream), else issued here (on
        the side stream, forked from the main stream, when overlapping)."""
        if self._dw_queue is not None:
            self._dw_queue.append((args, kw))
            return None
        if not self.overlap:
            return self._gemm(*args, **kw)
        check(self.lib.it_side_begin(self.h), "side stream")
        try:
            self._gemm(*args, **kw)
        finally:
            check(self.lib.it_side_end(self.h), "side stream")

    def _dw_flush(self):
        """The layer's queued weight gradients (on the side stream when overlapping): one
        it_gemm_group call with group_weight_grads, else one GEMM after the other."""
        q, self._dw_queue = self._dw_queue, None
        if not q:
            return
        if self.overlap:
            check(self.lib.it_side_begin(self.h), "side stream")
        try:
            if self.group_weight_grads:
                calls = (_lib.GemmCall * len(q))(*[self._call(*a[1:], **kw) for a, kw in q])
                check(self.lib.it_gemm_group(self.h, 0, 0, len(q), calls), "weight gradients")
            else:
                for args, kw in q:
                    self._gemm(*args, **kw)
        finally:
            if self.overlap:
                check(self.lib.it_side_end(self.h), "side stream")

    def _norm(self, x: Tensor, res: Optional[Tensor], gamma: Tensor, sum_out: Optional[Tensor], y: Tensor):
        T, H = self.s.tokens, self.s.hidden
        vp = lambda t: C.c_void_p(t.ptr) if t is not None else C.c_void_p(0)
        check(self.lib.it_rmsnorm_forward(self.h, 0, T, H, self.eps, vp(x), vp(res), vp(gamma), vp(sum_out), vp(y)),
              "rmsnorm")

    def _norm_bwd(self, dy: Tensor, x: Tensor, gamma: Tensor, gres: Optional[Tensor], dx: Tensor, dgamma: Tensor):
        T, H = self.s.tokens, self.s.hidden
        check(self.lib.it_rmsnorm_backward(self.h, T, H, self.eps, C.c_void_p(dy.ptr), C.c_void_p(x.ptr),
                                           C.c_void_p(gamma.ptr), C.c_void_p(gres.ptr) if gres is not None else None,
                                           C.c_void_p(dx.ptr), C.c_void_p(dgamma.ptr)), "rmsnorm_backward")

    def _rope(self, buf: Tensor, backward: bool):
        """Rotates the Q and K blocks of a [T, 3H] buffer in place (2 * heads heads per row)."""
        s = self.s
        check(self.lib.it_rope(self.h, 0, 0, s.batch, s.seq, 2 * s.heads, s.head_dim, self.rope_base, 0,
                               int(backward), C.c_void_p(buf.ptr), 3 * s.hidden, C.c_void_p(buf.ptr), 3 * s.hidden,
                               0), "rope")

    def _layouts(self):
        s = self.s
        qkv = _lib.AttnLayout(s.heads, s.seq * 3 * s.hidden, s.head_dim, 3 * s.hidden)
        o = _lib.AttnLayout(s.heads, s.seq * s.hidden, s.head_dim, s.hidden)
        return qkv, o

    # ---------------------------------------------------------------- the step
    def _forward_layer(self, l: int) -> None:
        s = self.s
        T, H, F = s.tokens, s.hidden, s.ffn
        L = s.layers
        # Q|K|V projection with RoPE applied to the Q and K columns in the GEMM's epilogue
        rope = _lib.Epilogue(flags=_lib.IT_EPI_ROPE, rope_base=self.rope_base, rope_seq=s.seq,
                             rope_head_dim=s.head_dim, rope_cols=2 * H, rope_offset=0)
        self._gemm("qkv", self.xn[l], self.Wqkv[l], self.QKV[l], False, True, T, 3 * H, H, epi=rope)
        qkv, o = self._layouts()
        q, k, v = (C.c_void_p(self.QKV[l].ptr + i * H * 4) for i in range(3))
        scale = 1.0 / math.sqrt(s.head_dim)
        bh = s.batch * s.heads
        if self.fused:
            st = self.lib.it_flash_attention_forward(self.h, 0, bh, s.seq, s.seq, s.head_dim, scale, 1,
                                                     C.byref(qkv), C.byref(qkv), C.byref(o), q, k, v,
                                                     C.c_void_p(self.O[l].ptr), C.c_void_p(self.lse[l].ptr))
        else:
            st = self.lib.it_attention_forward(self.h, 0, bh, s.seq, s.seq, s.head_dim, scale, 1, C.byref(qkv),
                                               C.byref(qkv), C.byref(o), q, k, v, C.c_void_p(self.Sc.ptr),
                                               C.c_void_p(self.Pw.ptr), C.c_void_p(self.O[l].ptr))
        check(st, "attention")
        self._gemm("wo", self.O[l], self.Wo[l], self.Y, False, True, T, H, H)
        # post = x + attn_out; x2 = ffn_norm(post)
        self._norm(self.xin[l], self.Y, self.ffn_norm[l], self.post[l], self.x2[l])
        epi = _lib.Epilogue(flags=_lib.IT_EPI_SWIGLU, B2=self.Wgu[l].ptr + F * H * 4,
                            gate_out=self.G[l].ptr, up_out=self.U[l].ptr)
        self._gemm("gate_up_swiglu", self.x2[l], self.Wgu[l], self.Hh[l], False, True, T, F, H, epi=epi)
        self._gemm("down", self.Hh[l], self.Wd[l], self.Z, False, True, T, H, F)
        # out = post + ffn_out, normed by the next layer's attention norm (or the final norm)
        if l + 1 < L:
            self._norm(self.post[l], self.Z, self.attn_norm[l + 1], self.xin[l + 1], self.xn[l + 1])
        else:
            self._norm(self.post[l], self.Z, self.final_norm, self.xin[L], self.Hf)

    def _backward_layer(self, l: int) -> None:
        s = self.s
        T, H, F = s.tokens, s.hidden, s.ffn
        g = self.g_out[l + 1]
        if (self.overlap and self.dw_fork == "layer") or self.group_weight_grads:
            self._dw_queue = []
        # FFN: down projection, SwiGLU, gate|up projection, ffn norm (+ residual)
        self._dw("down.dW", g, self.Hh[l], self.dWd[l], True, False, H, F, T)
        # dL/dh = g.Wd goes straight through the SwiGLU backward in the GEMM's epilogue into dGate|dUp
        swb = _lib.Epilogue(flags=_lib.IT_EPI_SWIGLU_BWD, gate_out=self.G[l].ptr, up_out=self.U[l].ptr)
        self._gemm("down.dX+swiglu_bwd", g, self.Wd[l], self.dGU[l], False, False, T, F, H, epi=swb)
        self._dw("gate_up.dW", self.dGU[l], self.x2[l], self.dWgu[l], True, False, 2 * F, H, T)
        self._gemm("gate_up.dX", self.dGU[l], self.Wgu[l], self.dX2, False, False, T, H, 2 * F)
        self._norm_bwd(self.dX2, self.post[l], self.ffn_norm[l], g, self.gpost[l], self.d_ffn_norm[l])
        # attention: output projection, attention backward, RoPE backward, QKV projection, attn norm
        gp = self.gpost[l]
        self._dw("wo.dW", gp, self.O[l], self.dWo[l], True, False, H, H, T)
        self._gemm("wo.dX", gp, self.Wo[l], self.dOp, False, False, T, H, H)
        qkv, o = self._layouts()
        q, k, v = (C.c_void_p(self.QKV[l].ptr + i * H * 4) for i in range(3))
        dq, dk, dv = (C.c_void_p(self.dQKV[l].ptr + i * H * 4) for i in range(3))
        scale = 1.0 / math.sqrt(s.head_dim)
        bh = s.batch * s.heads
        if self.fused:
            st = self.lib.it_flash_attention_backward(self.h, 0, bh, s.seq, s.head_dim, scale, 1, C.byref(qkv),
                                                      C.byref(qkv), C.byref(o), C.c_void_p(self.dOp.ptr), q, k, v,
                                                      C.c_void_p(self.O[l].ptr), C.c_void_p(self.lse[l].ptr),
                                                      dq, dk, dv)
        else:
            st = self.lib.it_attention_backward(self.h, 0, bh, s.seq, s.head_dim, scale, 1, C.byref(qkv),
                                                C.byref(qkv), C.byref(o), C.c_void_p(self.dOp.ptr), q, k, v,
                                                C.c_void_p(self.Sc.ptr), C.c_void_p(self.Pw.ptr),
                                                C.c_void_p(self.dP.ptr), C.c_void_p(self.dS.ptr), dq, dk, dv)
        check(st, "attention_backward")
        self._rope(self.dQKV[l], True)
        self._dw("qkv.dW", self.dQKV[l], self.xn[l], self.dWqkv[l], True, False, 3 * H, H, T)
        self._dw_flush()
        self._gemm("qkv.dX", self.dQKV[l], self.Wqkv[l], self.dXn, False, False, T, H, 3 * H)
        self._norm_bwd(self.dXn, self.xin[l], self.attn_norm[l], gp, self.g_out[l], self.d_attn_norm[l])

    def enqueue(self) -> None:
        """Issues one full step (forward, loss, backward, clip, Lion) on the context's stream."""
        s = self.s
        self._dw_queue = None  # a step interrupted mid-layer leaves no queued weight gradients
        T, H, V, L = s.tokens, s.hidden, s.vocab, s.layers
        check(self.lib.it_embedding_forward(self.h, 0, 0, T, H, V, C.c_void_p(self.emb.ptr), C.c_void_p(self.ids.ptr),
                                            C.c_void_p(self.xin[0].ptr)), "embedding")
        self._norm(self.xin[0], None, self.attn_norm[0], None, self.xn[0])
        for l in range(L):
            self._forward_layer(l)
        self._gemm("lm_head", self.Hf, self.E, self.logits, False, True, T, V, H)
        if self.xent_operand:
            check(self.lib.it_cross_entropy_stats(self.h, T, V, C.c_void_p(self.logits.ptr),
                                                  C.c_void_p(self.targets.ptr), C.c_void_p(self.losses.ptr),
                                                  C.c_void_p(self.ce_stats.ptr), C.c_void_p(self.loss.ptr)),
                  "cross_entropy_stats")
            xent = _lib.Epilogue(flags=_lib.IT_EPI_XENT_A, xent_stats=self.ce_stats.ptr,
                                 xent_targets=self.targets.ptr,
                                 xent_scale=float(np.float32(1.0) / np.float32(T)))
            self._dw("lm_head.dW", self.logits, self.Hf, self.dE, True, False, V, H, T, epi=xent)
            self._gemm("lm_head.dX", self.logits, self.E, self.dHf, False, False, T, H, V, epi=xent)
        else:
            check(self.lib.it_cross_entropy_fused(self.h, 0, T, V, C.c_void_p(self.logits.ptr),
                                                  C.c_void_p(self.targets.ptr), C.c_void_p(self.losses.ptr),
                                                  C.c_void_p(self.dlogits.ptr), C.c_void_p(self.loss.ptr)),
                  "cross_entropy_fused")
            self._dw("lm_head.dW", self.dlogits, self.Hf, self.dE, True, False, V, H, T)
            self._gemm("lm_head.dX", self.dlogits, self.E, self.dHf, False, False, T, H, V)
        self._norm_bwd(self.dHf, self.xin[L], self.final_norm, None, self.g_out[L], self.d_final_norm)
        for l in reversed(range(L)):
            self._backward_layer(l)
        check(self.lib.it_embedding_backward(self.h, T, H, V, C.c_void_p(self.g_out[0].ptr), C.c_void_p(self.ids.ptr),
                                             C.c_void_p(self.d_emb.ptr)), "embedding_backward")
        if self.overlap:
            check(self.lib.it_side_join(self.h), "side stream")
        n = len(self.grads)
        gp = (C.c_void_p * n)(*[t.ptr for t in self.grads])
        sz = (C.c_int64 * n)(*[t.numel() for t in self.grads])
        check(self.lib.it_grad_norm_clip(self.h, n, gp, sz, self.max_grad_norm, C.c_void_p(self.norm_clip.ptr)),
              "grad_norm")
        wp = (C.c_void_p * n)(*[t.ptr for t in self.params])
        mp = (C.c_void_p * n)(*[t.ptr for t in self.momentum])
        check(self.lib.it_lion_step(self.h, n, wp, mp, gp, sz, self.lr, self.beta1, self.beta2, self.wd,
                                    C.c_void_p(self.norm_clip.ptr + 4), C.c_void_p(self.lr_dev.ptr)), "lion")

    def step(self) -> None:
        """One step: the captured graph when there is one, eager launches otherwise."""
        if self.graph is not None:
            check(self.lib.it_graph_launch(self.h, self.graph), "graph launch")
        else:
            self.enqueue()

    def capture(self) -> None:
        """Captures one step into a HIP graph (run a step eagerly first so scratch is sized)."""
        check(self.lib.it_capture_begin(self.h), "capture")
        try:
            self.enqueue()
        finally:
            g = C.c_void_p()
            st = self.lib.it_capture_end(self.h, C.byref(g))
        check(st, "capture")
        self.graph = g

    def loss_value(self) -> float:
        return float(self.loss.as_f32_slice()[0])

    def grad_norm(self) -> float:
        return float(self.norm_clip.as_f32_slice()[0])

    def gemm_flops(self) -> float:
        """Dense-equivalent FLOPs of the step's contractions (attention counted as its GEMMs)."""
        s = self.s
        T, H, F, V, L = s.tokens, s.hidden, s.ffn, s.vocab, s.layers
        attn = 2.0 * s.batch * s.heads * s.seq * s.seq * s.head_dim
        per_layer_fwd = 2.0 * T * H * (3 * H + H + 2 * F + F) + 2 * attn
        per_layer_bwd = 2 * 2.0 * T * H * (3 * H + H + 2 * F + F) + 5 * attn
        return L * (per_layer_fwd + per_layer_bwd) + 3 * 2.0 * T * H * V

    # ---------------------------------------------------------------- checkpoints (IRON v2)
    def _named(self, tensors: List[Tensor]):
        """(embed, final_norm, E, layers) in the reference's names, from params-ordered tensors."""
        s = self.s
        H, F = s.hidden, s.ffn
        arrs = [t.numpy() for t in tensors]
        layers = []
        for l in range(s.layers):
            an, fn, qkv, wo, gu, wd = arrs[3 + 6 * l: 9 + 6 * l]
            layers.append({"wq": qkv[:H], "wk": qkv[H:2 * H], "wv": qkv[2 * H:], "wo": wo, "w_gate": gu[:F],
                           "w_up": gu[F:], "w_down": wd, "attn_norm": an, "ffn_norm": fn})
        return arrs[0], arrs[1], arrs[2], layers

    def save_checkpoint(self, path, step: int = 0, epoch: int = 0, best_val_loss: float = float("inf"),
                        with_optimizer: bool = True) -> None:
        """Writes the parameters (and the Lion momenta) as an IRON v2 file: Q|K|V and gate|up are
        split back into the reference's wq, wk, wv and w_gate, w_up; the untied LM head goes into the
        extension block (irontensor_amd.checkpoint)."""
        from . import checkpoint as ck
        s = self.s
        cfg = ck.ModelConfig(s.vocab, s.hidden, s.layers, s.heads, s.heads, s.ffn, self.eps, self.rope_base, s.seq,
                             False, 0)
        emb, fnorm, E, layers = self._named(self.params)
        w = ck.Weights(emb, layers, fnorm, E)
        opt = None
        if with_optimizer:
            m_emb, m_fn, m_E, m_layers = self._named(self.momentum)
            opt = ck.OptimizerState(m_emb, m_layers, m_fn, m_E)
        ck.save_model_weights(path, w, ck.Checkpoint(cfg, step, epoch, best_val_loss, self.lr, with_optimizer), opt)

    def load_checkpoint(self, path):
        """Loads an IRON v2 file written for this shape into the parameters (and momenta when the
        file has them; zeros otherwise). Returns the Checkpoint metadata."""
        from . import checkpoint as ck
        w, meta, opt = ck.load_model_weights(path)
        s, c = self.s, meta.config
        if (c.vocab_size, c.hidden_dim, c.num_layers, c.num_heads, c.intermediate_dim) != \
                (s.vocab, s.hidden, s.layers, s.heads, s.ffn) or c.num_kv_heads != c.num_heads:
            raise ValueError(f"checkpoint config {c} does not match the step's shape {s}")
        out = w.output_weight if w.output_weight is not None else w.embed_tokens

        def flat(embed, final_norm, output, layers):
            arrs = [embed, final_norm, output]
            for L in layers:
                arrs += [L["attn_norm"], L["ffn_norm"], np.concatenate([L["wq"], L["wk"], L["wv"]]), L["wo"],
                         np.concatenate([L["w_gate"], L["w_up"]]), L["w_down"]]
            return arrs

        def upload(dst: List[Tensor], arrs):
            for t, a in zip(dst, arrs):
                a = np.ascontiguousarray(a, np.float32)
                if list(a.shape) != t.shape():
                    raise ValueError(f"checkpoint tensor of shape {list(a.shape)} where {t.shape()} is expected")
                check(self.lib.it_memcpy_h2d(self.h, C.c_void_p(t.ptr), a.ctypes.data_as(C.c_void_p), a.nbytes),
                      "load checkpoint")

        upload(self.params, flat(w.embed_tokens, w.final_norm, out, w.layers))
        if opt is not None:
            o_out = opt.output_weight if opt.output_weight is not None else np.zeros_like(out)
            upload(self.momentum, flat(opt.embed, opt.final_norm, o_out, opt.layers))
        else:
            for m in self.momentum:
                check(self.lib.it_zero(self.h, C.c_void_p(m.ptr), m.byte_size()), "zero momentum")
        self.set_lr(meta.learning_rate)
        return meta

    def close(self) -> None:
        if self.graph is not None:
            self.lib.it_graph_destroy(self.graph)
            self.graph = None
