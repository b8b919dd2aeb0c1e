"""Pins the oracle's training-step ops (oracle/train_ref.c) before they judge the GPU: closed forms,
identities and finite differences, each chosen so that a plausible slip (a dropped term, a wrong
sign or index, a transposed operand) fails. Plants such slips to show the checks catch them."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth


def _fd(f, x, eps=1e-3):
    """Central finite differences of scalar f at float64 x."""
    g = np.zeros_like(x)
    it = np.nditer(x, flags=["multi_index"])
    for _ in it:
        i = it.multi_index
        xp, xm = x.copy(), x.copy()
        xp[i] += eps
        xm[i] -= eps
        g[i] = (f(xp) - f(xm)) / (2 * eps)
    return g


# ---------------------------------------------------------------- RMSNorm (src/shaders/norm.metal)

def test_rmsnorm_closed_forms(oracle):
    x = np.full((3, 8), 2.0, np.float32)
    y = oracle.rmsnorm(x, np.ones(8, np.float32), 0.0)
    assert np.allclose(y, 1.0, atol=1e-7)  # constant rows normalise to 1
    g = np.arange(1, 9, dtype=np.float32)
    assert np.allclose(oracle.rmsnorm(x, g, 0.0), g[None, :], atol=1e-6)
    x = synth.normal(1, (5, 64))
    ref = x / np.sqrt((x.astype(np.float64) ** 2).mean(-1, keepdims=True) + 1e-5) * g.mean()
    assert np.allclose(oracle.rmsnorm(x, np.full(64, g.mean(), np.float32), 1e-5), ref, rtol=1e-5, atol=1e-6)


def test_rmsnorm_backward_finite_differences(oracle):
    rows, dim, eps = 3, 6, 1e-5
    x = synth.normal(2, (rows, dim)).astype(np.float64)
    gamma = synth.normal(3, (dim,)).astype(np.float64)
    dy = synth.normal(4, (rows, dim)).astype(np.float64)

    def f(xx, gg):
        y = xx / np.sqrt((xx ** 2).mean(-1, keepdims=True) + eps) * gg
        return float((y * dy).sum())

    dx, dg = oracle.rmsnorm_backward(dy, x, gamma, eps)
    assert np.allclose(dx, _fd(lambda v: f(v, gamma), x), rtol=2e-3, atol=2e-4)
    assert np.allclose(dg, _fd(lambda v: f(x, v), gamma), rtol=2e-3, atol=2e-4)


# ---------------------------------------------------------------- RoPE (src/shaders/rope.metal)

def test_rope_identities(oracle):
    x = synth.normal(5, (2, 7, 3, 8))
    y = oracle.rope(x)
    assert np.allclose(y[:, 0], x[:, 0])  # position 0 is the identity
    # rotations preserve each pair's length
    assert np.allclose((y.reshape(-1, 2) ** 2).sum(-1), (x.reshape(-1, 2) ** 2).sum(-1), rtol=1e-5)
    back = oracle.rope(y, backward=True)
    assert np.allclose(back, x, atol=1e-5)  # the backward is the inverse rotation
    # pair i at position p: angle p * base^(-2i/d), rotation [[c, -s], [s, c]]
    p, i, d = 3, 2, 8
    a = p * 10000.0 ** (-2 * i / d)
    x0, x1 = x[0, p, 1, 2 * i], x[0, p, 1, 2 * i + 1]
    assert np.isclose(y[0, p, 1, 2 * i], x0 * np.cos(a) - x1 * np.sin(a), atol=1e-5)
    assert np.isclose(y[0, p, 1, 2 * i + 1], x0 * np.sin(a) + x1 * np.cos(a), atol=1e-5)


def test_rope_strided_rows(oracle):
    """The rotated block inside a wider row (the fused QKV buffer) equals the contiguous form and
    leaves the other columns alone."""
    b, s, h, d = 2, 5, 2, 8
    buf = synth.normal(6, (b, s, 3 * h * d))
    y = oracle.rope(buf, heads=h, head_dim=d)
    ref = oracle.rope(buf[:, :, : h * d].reshape(b, s, h, d))
    assert np.allclose(y[:, :, : h * d].reshape(b, s, h, d), ref)
    assert np.array_equal(y[:, :, h * d:], buf[:, :, h * d:])


# ---------------------------------------------------------------- embedding

def test_embedding_backward_is_the_transpose(oracle):
    vocab, dim, n = 11, 4, 9
    table = synth.normal(7, (vocab, dim))
    ids = synth.tokens(8, n, vocab)
    dy = synth.normal(9, (n, dim))
    out = oracle.embedding(table, ids)
    assert np.array_equal(out, table[ids])
    dw = oracle.embedding_backward(dy, ids, vocab)
    # <dW, W> == <dY, gather(W)> for any W
    assert np.isclose((dw.astype(np.float64) * table).sum(), (dy.astype(np.float64) * out).sum(), rtol=1e-5)
    unused = np.setdiff1d(np.arange(vocab), ids)
    assert np.all(dw[unused] == 0)


# ---------------------------------------------------------------- cross entropy (src/shaders/loss.metal)

def test_cross_entropy_closed_forms_and_gradient(oracle):
    mean, losses, grad = oracle.cross_entropy(np.zeros((4, 10), np.float32), np.array([0, 3, 9, 5]))
    assert np.allclose(losses, np.log(10), atol=1e-6) and np.isclose(mean, np.log(10), atol=1e-6)
    logits = synth.normal(10, (3, 7)).astype(np.float64)
    t = np.array([2, 0, 6])
    mean, losses, grad = oracle.cross_entropy(logits, t)
    assert np.allclose(grad.sum(-1), 0, atol=1e-7)  # softmax - onehot sums to zero per row

    def f(z):
        m = z.max(-1, keepdims=True)
        lse = (m + np.log(np.exp(z - m).sum(-1, keepdims=True)))[:, 0]
        return float((lse - z[np.arange(3), t]).mean())

    assert np.isclose(mean, f(logits), rtol=1e-6)
    assert np.allclose(grad, _fd(f, logits), rtol=1e-3, atol=1e-5)


# ---------------------------------------------------------------- Lion (src/shaders/lion.metal)

def test_lion_by_hand(oracle):
    w = np.array([1.0, -2.0, 0.5, 3.0], np.float32)
    m = np.array([0.1, -0.1, 0.0, 0.0], np.float32)
    g = np.array([1.0, 1.0, 0.0, -4.0], np.float32)
    lr, b1, b2, wd = 0.1, 0.9, 0.99, 0.01
    w2, m2 = oracle.lion(w, m, g, lr, b1, b2, wd)
    # direction uses beta2: 0.99*0.1+0.01*1 > 0; 0.99*-0.1+0.01*1 < 0; exactly 0 -> 0; < 0
    dirs = np.array([1.0, -1.0, 0.0, -1.0], np.float32)
    assert np.allclose(w2, w - lr * dirs - lr * wd * w, atol=1e-7)
    assert np.allclose(m2, b1 * m + (1 - b1) * g, atol=1e-7)
    w3, _ = oracle.lion(w, m, g, lr, b1, b2, wd, scale=0.5)  # clipping scales g first
    assert np.allclose(w3, oracle.lion(w, m, g * np.float32(0.5), lr, b1, b2, wd)[0])


def test_sum_squares(oracle):
    x = synth.normal(11, (1000,))
    assert np.isclose(oracle.sum_squares(x), float((x.astype(np.float64) ** 2).sum()), rtol=1e-12)


# ---------------------------------------------------------------- planted slips are caught

def test_planted_slips_fail(oracle):
    x = synth.normal(12, (2, 6)).astype(np.float64)
    gamma = synth.normal(13, (6,)).astype(np.float64)
    dy = synth.normal(14, (2, 6)).astype(np.float64)
    dx, _ = oracle.rmsnorm_backward(dy, x, gamma, 1e-5)
    s = 1 / np.sqrt((x ** 2).mean(-1, keepdims=True) + 1e-5)
    dropped = dy * gamma * s  # the s^3 * x * dot term dropped
    assert not np.allclose(dx, dropped, rtol=2e-3, atol=2e-4)
    y = synth.normal(15, (1, 4, 1, 4))
    wrong_sign = oracle.rope(y, backward=False)
    assert not np.allclose(oracle.rope(wrong_sign, backward=False), y, atol=1e-5)  # forward twice != identity
    _, _, grad = oracle.cross_entropy(synth.normal(16, (2, 5)), np.array([1, 4]))
    assert not np.allclose(grad.sum(-1) + 1.0 / 2, 0, atol=1e-7)  # a missing onehot would sum to 1/rows


def test_rope_theta_is_the_correctly_rounded_power():
    """The oracle's theta uses the host powf; the GPU kernel rounds a double-precision power once.
    They agree when the host powf is correctly rounded at these arguments, which this checks for
    every pair index of the head sizes in use (a one-ulp theta shows after the position multiply)."""
    import ctypes
    libm = ctypes.CDLL("libm.so.6")
    libm.powf.restype, libm.powf.argtypes = ctypes.c_float, [ctypes.c_float, ctypes.c_float]
    for d in (2, 16, 32, 64, 128, 256):
        for i in range(d // 2):
            e = np.float32(np.float32(2 * i) / np.float32(d))
            assert np.float32(libm.powf(10000.0, float(e))) == np.float32(np.power(10000.0, np.float64(e)))


# ---------------------------------------------------------------- fused RMSNorm + projection

def test_fused_rmsnorm_linear_oracle(oracle):
    """Against rmsnorm then x.W^T in float64, the reference's own test data
    (src/ops/fused_rmsnorm_linear.rs:244-276, tolerance 1e-3 there) and two planted slips."""
    rows, hidden, out_f = 4, 64, 32
    x = ((np.arange(rows * hidden) % 100) - 50.0).astype(np.float32).reshape(rows, hidden) * np.float32(0.01)
    g = (1.0 + np.sin(np.arange(hidden, dtype=np.float64)) * 0.1).astype(np.float32)
    w = ((np.arange(out_f * hidden) % 200) - 100.0).astype(np.float32).reshape(out_f, hidden) * np.float32(0.001)
    got = oracle.fused_rmsnorm_linear(x, g, w, 1e-5)
    x64 = x.astype(np.float64)
    ref = (x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5) * g) @ w.astype(np.float64).T
    assert np.max(np.abs(got - ref)) <= 1e-6 * np.max(np.abs(ref)) + 1e-7
    assert np.max(np.abs(got - ref)) < 1e-3
    no_gamma = (x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5)) @ w.astype(np.float64).T
    assert np.max(np.abs(no_gamma - got)) > 1e-3
    no_inv = (x64 * g) @ w.astype(np.float64).T
    assert np.max(np.abs(no_inv - got)) > 1e-3


# ---------------------------------------------------------------- fused linear + cross entropy

def _flce_f64(h, w, t):
    h64, w64 = h.astype(np.float64), w.astype(np.float64)
    logits = h64 @ w64.T
    valid = (t >= 0) & (t < w.shape[0])
    m = logits.max(1, keepdims=True)
    lse = (m + np.log(np.exp(logits - m).sum(1, keepdims=True)))[:, 0]
    loss = np.where(valid, lse - logits[np.arange(len(t)), np.where(valid, t, 0)], 0.0)
    p = np.exp(logits - lse[:, None])
    p[np.arange(len(t))[valid], t[valid]] -= 1.0
    p[~valid] = 0.0
    n = max(int(valid.sum()), 1)
    return loss.sum() / n, loss, (p @ w64) / n, p.T @ h64


def test_fused_linear_cross_entropy_oracle(oracle):
    """Against the float64 composition logits -> cross entropy -> products, with ignored rows; the
    gradients against finite differences of the mean loss (grad_weight is the unscaled sum, so it
    is grad of the mean times the valid count); the reference's own comparison case
    (src/ops/fused_linear_cross_entropy.rs:389-451, tolerance 1e-3 there)."""
    h = synth.normal(30, (12, 16), std=0.7)
    w = synth.normal(31, (40, 16), std=0.5)
    t = synth.tokens(32, 12, 40).astype(np.int32)
    t[[2, 7]] = -100
    mean, losses, gh, gw = oracle.fused_linear_cross_entropy(h, w, t)
    rm, rl, rgh, rgw = _flce_f64(h, w, t)
    assert abs(mean - rm) <= 1e-6 * abs(rm)
    assert np.allclose(losses, rl, rtol=1e-5, atol=1e-6)
    assert np.allclose(gh, rgh, rtol=1e-4, atol=1e-6) and np.allclose(gw, rgw, rtol=1e-4, atol=1e-6)
    assert not gh[[2, 7]].any()

    def f_h(hh):
        return _flce_f64(hh, w, t)[0]

    def f_w(ww):
        return _flce_f64(h, ww, t)[0]

    n_valid = int(((t >= 0) & (t < 40)).sum())
    assert np.allclose(gh, _fd(f_h, h.astype(np.float64), 1e-4), rtol=1e-3, atol=1e-6)
    assert np.allclose(gw / n_valid, _fd(f_w, w.astype(np.float64), 1e-4), rtol=1e-3, atol=1e-6)
    # the reference's case: hidden sin(0.01 i) * 0.5, weight cos(0.02 i) * 0.3, targets 7i mod 64
    h2 = (np.sin(np.arange(8 * 32) * 0.01) * 0.5).astype(np.float32).reshape(8, 32)
    w2 = (np.cos(np.arange(64 * 32) * 0.02) * 0.3).astype(np.float32).reshape(64, 32)
    t2 = ((np.arange(8) * 7) % 64).astype(np.int32)
    m2, _, gh2, _ = oracle.fused_linear_cross_entropy(h2, w2, t2)
    sm, _, sgrad = oracle.cross_entropy(oracle.gemm_f32(h2, w2, trans_b=True), t2.astype(np.uint32))
    assert abs(m2 - sm) < 1e-3 and np.max(np.abs(gh2 - oracle.gemm_f32(sgrad, w2))) < 1e-3
