"""CPU ORACLE for one full training step -- test infrastructure only (tests/, smoke(), bench.py's
cpu_baseline may use it; the product never does).

Composes the oracle's restated kernels (ref.c, train_ref.c) in the reference trainer's order:
src/train/forward.rs:79-212 (layer forward: attn norm, Q/K/V projections, RoPE on Q and K, causal
attention, output projection, residual, ffn norm, gate/up, SwiGLU, down, residual),
src/train/trainer/train_step.rs:176-236 (final norm, logits, cross_entropy_fused, LM-head
backward, final-norm backward, layers in reverse), src/train/backward.rs:21-177 (layer backward),
train_step.rs:79 (embedding backward) and :395-460 (global L2 norm, clip, Lion on every
parameter). Weight shapes are the reference's [out, in]; Q|K|V and gate|up are kept stacked
([3H, H], [2F, H]) as the GPU step stores them, which changes nothing in the arithmetic of each
projection except that the three (two) input-gradient products are summed by one contraction.
Pinned by tests/test_oracle_train_step.py (finite differences of the loss on a small model).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Dict, List

import numpy as np

from . import (attention_bwd_bhsd, attention_fwd_bhsd, cross_entropy, embedding, embedding_backward,
               gemm_f32, lion, rmsnorm, rmsnorm_backward, rope, sum_squares, swiglu, swiglu_backward)


@dataclass(frozen=True)
class Hyper:
    eps: float = 1e-5
    rope_base: float = 10000.0
    lr: float = 3e-4
    beta1: float = 0.9
    beta2: float = 0.99
    weight_decay: float = 0.1
    max_grad_norm: float = 1.0


# Parameter order of the GPU step: emb, final_norm, E, then per layer
# attn_norm, ffn_norm, Wqkv, Wo, Wgu, Wd.
LAYER_KEYS = ("attn_norm", "ffn_norm", "Wqkv", "Wo", "Wgu", "Wd")


def param_list(p: Dict) -> List[np.ndarray]:
    out = [p["emb"], p["final_norm"], p["E"]]
    for l in range(len(p["Wqkv"])):
        out += [p[k][l] for k in LAYER_KEYS]
    return out


def _heads(x, b, s, h, d):
    """[T, h*d] -> [b*h, s, d]"""
    return np.ascontiguousarray(x.reshape(b, s, h, d).transpose(0, 2, 1, 3)).reshape(b * h, s, d)


def _unheads(x, b, s, h, d):
    return np.ascontiguousarray(x.reshape(b, h, s, d).transpose(0, 2, 1, 3)).reshape(b * s, h * d)


def forward(p: Dict, ids, shape, hp: Hyper = Hyper(), threads=None):
    """Returns (logits, cache)."""
    b, s, h, d = shape.batch, shape.seq, shape.heads, shape.head_dim
    H, F = shape.hidden, shape.ffn
    scale = 1.0 / np.sqrt(d)
    x = embedding(p["emb"], ids)
    cache = {"xin": [x], "layers": []}
    for l in range(len(p["Wqkv"])):
        xin = cache["xin"][-1]
        xn = rmsnorm(xin, p["attn_norm"][l], hp.eps)
        qkv = gemm_f32(xn, p["Wqkv"][l], trans_b=True, threads=threads)
        qkv = rope(qkv.reshape(b, s, 3 * H), hp.rope_base, 0, heads=2 * h, head_dim=d).reshape(b * s, 3 * H)
        q, k, v = (_heads(qkv[:, i * H:(i + 1) * H], b, s, h, d) for i in range(3))
        o, _ = attention_fwd_bhsd(q, k, v, scale, True, threads=threads)
        O = _unheads(o, b, s, h, d)
        post = xin + gemm_f32(O, p["Wo"][l], trans_b=True, threads=threads)
        x2 = rmsnorm(post, p["ffn_norm"][l], hp.eps)
        gate = gemm_f32(x2, p["Wgu"][l][:F], trans_b=True, threads=threads)
        up = gemm_f32(x2, p["Wgu"][l][F:], trans_b=True, threads=threads)
        hh = swiglu(gate, up)
        out = post + gemm_f32(hh, p["Wd"][l], trans_b=True, threads=threads)
        cache["layers"].append(dict(xn=xn, qkv=qkv, q=q, k=k, v=v, O=O, post=post, x2=x2, gate=gate, up=up, hh=hh))
        cache["xin"].append(out)
    hf = rmsnorm(cache["xin"][-1], p["final_norm"], hp.eps)
    cache["hf"] = hf
    return gemm_f32(hf, p["E"], trans_b=True, threads=threads), cache


def loss(p: Dict, ids, targets, shape, hp: Hyper = Hyper(), threads=None) -> float:
    logits, _ = forward(p, ids, shape, hp, threads)
    return cross_entropy(logits, targets)[0]


def gradients(p: Dict, ids, targets, shape, hp: Hyper = Hyper(), threads=None):
    """Returns (mean loss, grads dict keyed like params, logits)."""
    b, s, h, d = shape.batch, shape.seq, shape.heads, shape.head_dim
    H, F, V = shape.hidden, shape.ffn, shape.vocab
    L = len(p["Wqkv"])
    scale = 1.0 / np.sqrt(d)
    logits, c = forward(p, ids, shape, hp, threads)
    mean, _, dlogits = cross_entropy(logits, targets)
    g = {k: [None] * L for k in LAYER_KEYS}
    g["E"] = gemm_f32(dlogits, c["hf"], trans_a=True, threads=threads)
    dhf = gemm_f32(dlogits, p["E"], threads=threads)
    grad, g["final_norm"] = rmsnorm_backward(dhf, c["xin"][L], p["final_norm"], hp.eps)
    for l in reversed(range(L)):
        cl = c["layers"][l]
        g["Wd"][l] = gemm_f32(grad, cl["hh"], trans_a=True, threads=threads)
        dhh = gemm_f32(grad, p["Wd"][l], threads=threads)
        dgate, dup = swiglu_backward(dhh, cl["gate"], cl["up"])
        dgu = np.concatenate([dgate, dup], axis=1)
        g["Wgu"][l] = gemm_f32(dgu, cl["x2"], trans_a=True, threads=threads)
        dx2 = gemm_f32(dgate, p["Wgu"][l][:F], threads=threads) + gemm_f32(dup, p["Wgu"][l][F:], threads=threads)
        dpost, g["ffn_norm"][l] = rmsnorm_backward(dx2, cl["post"], p["ffn_norm"][l], hp.eps)
        gpost = grad + dpost
        g["Wo"][l] = gemm_f32(gpost, cl["O"], trans_a=True, threads=threads)
        dO = gemm_f32(gpost, p["Wo"][l], threads=threads)
        dq, dk, dv = attention_bwd_bhsd(_heads(dO, b, s, h, d), cl["q"], cl["k"], cl["v"], scale, True,
                                        threads=threads)
        dqkv = np.concatenate([_unheads(t, b, s, h, d) for t in (dq, dk, dv)], axis=1)
        dqkv = rope(dqkv.reshape(b, s, 3 * H), hp.rope_base, 0, backward=True, heads=2 * h,
                    head_dim=d).reshape(b * s, 3 * H)
        g["Wqkv"][l] = gemm_f32(dqkv, cl["xn"], trans_a=True, threads=threads)
        dxn = sum(gemm_f32(dqkv[:, i * H:(i + 1) * H], p["Wqkv"][l][i * H:(i + 1) * H], threads=threads)
                  for i in range(3))
        dxin, g["attn_norm"][l] = rmsnorm_backward(dxn, c["xin"][l], p["attn_norm"][l], hp.eps)
        grad = gpost + dxin
    g["emb"] = embedding_backward(grad, ids, V)
    return mean, g, logits


def train_step(p: Dict, momentum: List[np.ndarray], ids, targets, shape, hp: Hyper = Hyper(), threads=None):
    """One full step. Returns dict(loss, grads, norm, clip, params (updated), momentum (updated))."""
    mean, g, _ = gradients(p, ids, targets, shape, hp, threads)
    glist = param_list(g)
    norm = np.float32(np.sqrt(sum(sum_squares(x) for x in glist)))
    clip = np.float32(hp.max_grad_norm) / norm if norm > np.float32(hp.max_grad_norm) else np.float32(1.0)
    new_p, new_m = [], []
    for w, m, gr in zip(param_list(p), momentum, glist):
        w2, m2 = lion(w, m, gr, hp.lr, hp.beta1, hp.beta2, hp.weight_decay, scale=float(clip))
        new_p.append(w2)
        new_m.append(m2)
    return dict(loss=mean, grads=glist, norm=float(norm), clip=float(clip), params=new_p, momentum=new_m)
