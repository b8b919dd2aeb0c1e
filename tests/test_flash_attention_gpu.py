"""GPU parity of the fused (flash) attention kernels, head_dim 64, against the oracle's restatements
of ops::attention and attention_backward_recompute (src/ops/attention.rs:286-377,544-621,
src/train/helpers.rs:120-193). Same bars as the materialised path: FP32 normwise 1e-5, BF16 relative
Frobenius 1e-2 against the f32 oracle on the unrounded inputs. Sequence lengths that are not
multiples of the 64-row tile exercise the masked edges."""
from __future__ import annotations

import numpy as np
import pytest

from irontensor_amd import synth
from tests.numerics import BF16_FROB_TOL, FP32_TOL, frob_rel, normwise_rel

pytestmark = pytest.mark.gpu

D = 64


def _t(it, x):
    return it.Tensor.from_f32_slice(x, x.shape)


def _softmax_f64(q, k, scale, causal):
    """float64 scores and row log-sum-exp for [BH, Sq, D] x [BH, Skv, D]."""
    s = q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2) * scale
    if causal:
        s = np.where(np.triu(np.ones(s.shape[-2:], bool), 1), -np.inf, s)
    mx = s.max(-1, keepdims=True)
    e = np.exp(s - mx)
    return e / e.sum(-1, keepdims=True), (mx + np.log(e.sum(-1, keepdims=True)))[..., 0]


@pytest.mark.parametrize("fill,b,s,h,causal", [
    # the fills of src/ops/attention.rs:623-711 at head_dim 64
    ("simple", 1, 4, 2, False),
    ("causal", 1, 4, 1, True),
    ("larger", 2, 16, 4, True),
])
def test_flash_reference_fills(it, oracle, fill, b, s, h, causal):
    n = b * s * h * D
    i = np.arange(n, dtype=np.float32)
    if fill == "simple":
        q, k, v = i * np.float32(0.1) - 3, i * np.float32(0.1) - 2, i * np.float32(0.1) - 1
    elif fill == "causal":
        q = k = v = (i + 1) * np.float32(0.1)
    else:
        q = k = v = ((np.arange(n) % 100).astype(np.float32) - 50) * np.float32(0.01)
    q, k, v = (x.reshape(b, s, h, D).astype(np.float32) for x in (q, k, v))
    out = it.flash_attention(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
    ref = oracle.attention_bshd(q, k, v, causal)
    assert normwise_rel(out, ref) <= FP32_TOL


@pytest.mark.parametrize("b,s,h,causal", [(2, 100, 3, True), (2, 100, 3, False), (1, 257, 2, True)])
def test_flash_bshd_matches_oracle(it, oracle, b, s, h, causal):
    print(f"[flash bshd] b={b} s={s} h={h} causal={causal}", flush=True)
    q, k, v = (synth.normal(50 + i, (b, s, h, D)) for i in range(3))
    out = it.flash_attention(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
    ref = oracle.attention_bshd(q, k, v, causal)
    assert normwise_rel(out, ref) <= FP32_TOL
    # the materialised path agrees as well
    mat = it.attention(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
    assert normwise_rel(out, mat) <= FP32_TOL


def test_flash_kv_length_differs(it):
    b, sq, skv, h = 2, 70, 130, 3
    q = synth.normal(1, (b, sq, h, D))
    k = synth.normal(2, (b, skv, h, D))
    v = synth.normal(3, (b, skv, h, D))
    out = it.flash_attention(_t(it, q), _t(it, k), _t(it, v), False).numpy()
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))  # noqa: E731
    p, _ = _softmax_f64(t(q), t(k), 1 / np.sqrt(D), False)
    ref = (p @ t(v).astype(np.float64)).transpose(0, 2, 1, 3)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_empty_and_zero_kv(it):
    z = it.Tensor.zeros([1, 0, 2, D])
    assert it.flash_attention(z, z, z, False).shape() == [1, 0, 2, D]
    q = it.Tensor.from_f32_slice(synth.normal(4, (1, 3, 2, D)), [1, 3, 2, D])
    kv = it.Tensor.zeros([1, 0, 2, D])
    out = it.flash_attention(q, kv, kv, False).numpy()
    assert out.shape == (1, 3, 2, D) and np.all(out == 0)


@pytest.mark.parametrize("causal", [True, False])
def test_flash_forward_bhsd_o_and_lse(it, oracle, causal):
    b, h, s = 2, 4, 200
    q, k, v = (synth.normal(20 + i, (b, h, s, D)) for i in range(3))
    o, lse = it.flash_attention_forward_bhsd(*(_t(it, x) for x in (q, k, v)), causal=causal)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(D), causal)
    assert normwise_rel(o.numpy(), ro) <= FP32_TOL
    _, rl = _softmax_f64(q.reshape(b * h, s, D), k.reshape(b * h, s, D), 1 / np.sqrt(D), causal)
    assert np.max(np.abs(lse.numpy().astype(np.float64) - rl)) < 1e-5 * max(1.0, np.max(np.abs(rl)))


@pytest.mark.parametrize("b,h,s,causal", [(2, 4, 16, True), (2, 3, 200, True), (1, 2, 130, False),
                                          (4, 4, 256, True), (4, 8, 640, True)])
def test_flash_backward_f32(it, oracle, b, h, s, causal):
    """(2,4,16) is the shape family of src/train/helpers.rs:435-494 at head_dim 64; (4,4,256) is a
    quarter of one TINY layer; 200 and 130 leave partial tiles. Grids of up to 256 blocks run each
    block's 16-row jobs as two waves that split every tile; (4,8,640) has 320 blocks and runs the
    one-wave form."""
    print(f"[flash bwd f32] {b}x{h}x{s} causal={causal}", flush=True)
    q, k, v, do = (synth.normal(10 + i, (b, h, s, D)) for i in range(4))
    tq, tk, tv, tdo = (_t(it, x) for x in (q, k, v, do))
    rq, rk, rv = oracle.attention_bwd_bhsd(do, q, k, v, 1 / np.sqrt(D), causal)
    got = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal)
    o, lse = it.flash_attention_forward_bhsd(tq, tk, tv, causal=causal)
    saved = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, o=o, lse=lse)
    for name, g, sv, ref in zip("QKV", got, saved, (rq, rk, rv)):
        gg, ss = g.numpy(), sv.numpy()
        assert normwise_rel(gg, ref) <= FP32_TOL, name
        assert np.array_equal(gg, ss), name  # the recompute is the same forward kernel


def test_flash_backward_deterministic(it):
    b, h, s = 2, 4, 300
    q, k, v, do = (_t(it, synth.normal(60 + i, (b, h, s, D))) for i in range(4))
    first = [x.numpy() for x in it.flash_attention_backward(do, q, k, v)]
    for _ in range(2):
        again = [x.numpy() for x in it.flash_attention_backward(do, q, k, v)]
        for a, c in zip(first, again):
            assert np.array_equal(a, c)


def test_flash_bf16_forward_backward(it, oracle):
    """BASELINE config 3 at 1/16 of the batch (1 x 8 heads x 1024 x 64)."""
    b, h, s = 1, 8, 1024
    q, k, v, do = (synth.normal(30 + i, (b, h, s, D)) for i in range(4))
    tq, tk, tv, tdo = (it.Tensor.from_f32_as_bf16(x, x.shape) for x in (q, k, v, do))
    o, lse = it.flash_attention_forward_bhsd(tq, tk, tv, causal=True, scale=0.125)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 0.125, True)
    err_o = frob_rel(o.numpy(), ro)
    dq, dk, dv = it.flash_attention_backward(tdo, tq, tk, tv, causal=True, scale=0.125, o=o, lse=lse)
    rq, rk, rv = oracle.attention_bwd_bhsd(do, q, k, v, 0.125, True)
    errs = [frob_rel(x.numpy(), r) for x, r in ((dq, rq), (dk, rk), (dv, rv))]
    print(f"[flash bf16] frob O {err_o:.3e} dQ {errs[0]:.3e} dK {errs[1]:.3e} dV {errs[2]:.3e}", flush=True)
    assert err_o <= BF16_FROB_TOL
    assert max(errs) <= BF16_FROB_TOL


def test_flash_bf16_full_size(it, oracle):
    """Config 3 at full size [16,8,1024,64]: the fused forward and backward on all 128 heads, with
    three heads checked against the oracle and every output finite."""
    b, h, s = 16, 8, 1024
    q, k, v, do = (synth.normal(70 + i, (b, h, s, D)) for i in range(4))
    tq, tk, tv, tdo = (it.Tensor.from_f32_as_bf16(x, x.shape) for x in (q, k, v, do))
    o, lse = it.flash_attention_forward_bhsd(tq, tk, tv, causal=True, scale=0.125)
    dq, dk, dv = it.flash_attention_backward(tdo, tq, tk, tv, causal=True, scale=0.125, o=o, lse=lse)
    flat = lambda x: x.reshape(b * h, s, D)  # noqa: E731
    outs = [flat(x.numpy()) for x in (o, dq, dk, dv)]
    for x in outs:
        assert np.all(np.isfinite(x))
    pick = [0, 77, 127]
    sub = lambda x: flat(x)[pick]  # noqa: E731
    ro, _ = oracle.attention_fwd_bhsd(sub(q), sub(k), sub(v), 0.125, True)
    refs = (ro,) + tuple(oracle.attention_bwd_bhsd(sub(do), sub(q), sub(k), sub(v), 0.125, True))
    for got, ref in zip(outs, refs):
        assert frob_rel(got[pick], ref) <= BF16_FROB_TOL


def test_flash_rejects_other_head_dims(it):
    x = it.Tensor.from_f32_slice(synth.normal(5, (1, 8, 2, 32)), [1, 8, 2, 32])
    with pytest.raises(it.TensorError, match="head_dim must be 64"):
        it.flash_attention(x, x, x, False)
