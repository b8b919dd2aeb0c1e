"""Pins the oracle's full training step (oracle/train_step.py) before it judges the GPU step: every
parameter gradient against central finite differences of the oracle's own loss on a small model,
so a wiring slip (a missing residual gradient, RoPE applied the wrong way, a transposed weight,
the wrong norm input) fails; plus the clip rule and the embedding-gradient identity."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth
from irontensor_amd.step import ModelShape

SMALL = ModelShape("small", 2, 8, 2, 4, 12, 11, 2, 5)


def _params(seed=100, std=0.3):
    s = SMALL
    H, F, V, L = s.hidden, s.ffn, s.vocab, s.layers
    k = iter(range(seed, seed + 1000))
    n = lambda shape, sd=std: synth.normal(next(k), shape, std=sd)
    return {
        "emb": n((V, H), 1.0), "E": n((V, H)), "final_norm": 1 + n((H,), 0.1),
        "attn_norm": [1 + n((H,), 0.1) for _ in range(L)], "ffn_norm": [1 + n((H,), 0.1) for _ in range(L)],
        "Wqkv": [n((3 * H, H)) for _ in range(L)], "Wo": [n((H, H)) for _ in range(L)],
        "Wgu": [n((2 * F, H)) for _ in range(L)], "Wd": [n((H, F)) for _ in range(L)],
    }


def _batch():
    s = SMALL
    stream = synth.tokens(7, s.batch * (s.seq + 1), s.vocab).reshape(s.batch, s.seq + 1)
    return stream[:, :-1].ravel(), stream[:, 1:].ravel()


def _entries(p):
    yield "emb", None, p["emb"]
    yield "E", None, p["E"]
    yield "final_norm", None, p["final_norm"]
    for key in ("attn_norm", "ffn_norm", "Wqkv", "Wo", "Wgu", "Wd"):
        for l in range(SMALL.layers):
            yield key, l, p[key][l]


def test_oracle_step_gradients_match_finite_differences(oracle):
    from oracle import train_step as ts
    p = _params()
    ids, tg = _batch()
    _, g, _ = ts.gradients(p, ids, tg, SMALL)
    rng = np.random.default_rng(0)
    eps = 1e-2
    for key, l, w in _entries(p):
        gw = g[key] if l is None else g[key][l]
        flat = np.abs(gw).ravel()
        picks = list(np.argsort(flat)[-3:]) + list(rng.integers(0, flat.size, 2))
        for idx in picks:
            i = np.unravel_index(idx, w.shape)
            orig = w[i]
            w[i] = orig + eps
            lp = ts.loss(p, ids, tg, SMALL)
            w[i] = orig - eps
            lm = ts.loss(p, ids, tg, SMALL)
            w[i] = orig
            fd = (lp - lm) / (2 * eps)
            assert abs(fd - gw[i]) <= 3e-4 + 0.01 * abs(gw[i]), (key, l, i, fd, gw[i])


def test_oracle_step_planted_slip_is_caught(oracle):
    """Dropping the norms' input gradients (a missing term) moves the projection gradients far beyond
    the finite-difference tolerance."""
    from oracle import train_step as ts
    p = _params()
    ids, tg = _batch()
    _, g, _ = ts.gradients(p, ids, tg, SMALL)
    orig = ts.rmsnorm_backward

    def broken(dy, x, gamma, eps=1e-5):
        dx, dg = orig(dy, x, gamma, eps)
        return dx * 0.0, dg

    ts.rmsnorm_backward = broken
    try:
        _, gb, _ = ts.gradients(p, ids, tg, SMALL)
    finally:
        ts.rmsnorm_backward = orig
    diff = np.max(np.abs(gb["Wqkv"][0] - g["Wqkv"][0]))
    assert diff > 10 * (3e-4 + 0.01 * np.max(np.abs(g["Wqkv"][0])))


def test_oracle_step_clip_and_lion(oracle):
    from oracle import train_step as ts
    p = _params()
    ids, tg = _batch()
    mom = [np.zeros_like(w) for w in ts.param_list(p)]
    hp = ts.Hyper(max_grad_norm=1e-3)
    out = ts.train_step(p, mom, ids, tg, SMALL, hp)
    norm = np.sqrt(sum(float((x.astype(np.float64) ** 2).sum()) for x in out["grads"]))
    assert abs(out["norm"] - norm) <= 1e-6 * norm
    assert out["clip"] == np.float32(1e-3) / np.float32(out["norm"])
    # zero momentum: m = (1 - beta1) * g * clip, and the step direction is sign(g)
    for w, w2, m2, gr in zip(ts.param_list(p), out["params"], out["momentum"], out["grads"]):
        gs = gr * np.float32(out["clip"])
        assert np.allclose(m2, np.float32(1 - hp.beta1) * gs, rtol=1e-6, atol=0)
        assert np.allclose(w2, w - hp.lr * np.sign(gs) - hp.lr * hp.weight_decay * w, rtol=1e-6, atol=1e-9)
