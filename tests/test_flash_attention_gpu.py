"""GPU parity of the fused (flash) attention entry points against the oracle's restatements of
ops::attention and attention_backward_recompute (src/ops/attention.rs:286-377,544-621,
src/train/helpers.rs:120-193), and of the reference's flash_attention contract
(src/ops/flash_attention.rs:76-193: [batch, heads, seq, head_dim], head_dim <= 128) with its own
three tests ported. Same bars as the materialised path: FP32 normwise 1e-5, BF16 relative Frobenius
1e-2 against the f32 oracle on the unrounded inputs. Sequence lengths that are not multiples of the
64-row (FP32) or 128-row (BF16) tile exercise the masked edges."""
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
    out = it.flash_attention_bshd(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
    ref = oracle.attention_bshd(q, k, v, causal)
    assert normwise_rel(out, ref) <= FP32_TOL


@pytest.mark.parametrize("b,s,h,causal", [(2, 100, 3, True), (2, 100, 3, False), (1, 257, 2, True)])
def test_flash_bshd_matches_oracle(it, oracle, b, s, h, causal):
    print(f"[flash bshd] b={b} s={s} h={h} causal={causal}", flush=True)
    q, k, v = (synth.normal(50 + i, (b, s, h, D)) for i in range(3))
    out = it.flash_attention_bshd(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
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
    out = it.flash_attention_bshd(_t(it, q), _t(it, k), _t(it, v), False).numpy()
    t = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))  # noqa: E731
    p, _ = _softmax_f64(t(q), t(k), 1 / np.sqrt(D), False)
    ref = (p @ t(v).astype(np.float64)).transpose(0, 2, 1, 3)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_empty_and_zero_kv(it):
    z = it.Tensor.zeros([1, 0, 2, D])
    assert it.flash_attention_bshd(z, z, z, False).shape() == [1, 0, 2, D]
    q = it.Tensor.from_f32_slice(synth.normal(4, (1, 3, 2, D)), [1, 3, 2, D])
    kv = it.Tensor.zeros([1, 0, 2, D])
    out = it.flash_attention_bshd(q, kv, kv, False).numpy()
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




# ------------------------------------------------ the reference's flash_attention contract, [B,H,S,D]

def _sin_fill(n, step, amp):
    """(i * step).sin() * amp in f32, as the reference's flash tests fill Q = K = V."""
    return (np.sin(np.arange(n, dtype=np.float32) * np.float32(step)) * np.float32(amp)).astype(np.float32)


def _to_bshd(x):
    return np.ascontiguousarray(x.transpose(0, 2, 1, 3))


@pytest.mark.parametrize("causal", [False, True])
def test_flash_attention_matches_standard(it, oracle, causal):
    """src/ops/flash_attention.rs:241-300: batch 2, heads 4, seq 32, head_dim 16, Q = K = V =
    sin(0.1 i) / 2; flash_attention against ops::attention on the transposed tensors (the
    reference's bar: max |diff| < 1e-3) and against the oracle (normwise 1e-5)."""
    b, h, s, d = 2, 4, 32, 16
    x = _sin_fill(b * h * s * d, 0.1, 0.5).reshape(b, h, s, d)
    out = it.flash_attention(_t(it, x), _t(it, x), _t(it, x), causal).numpy()
    assert out.shape == (b, h, s, d)
    xs = _to_bshd(x)
    std = _to_bshd(it.attention(_t(it, xs), _t(it, xs), _t(it, xs), causal).numpy())
    assert np.max(np.abs(out - std)) < 1e-3
    ref, _ = oracle.attention_fwd_bhsd(x, x, x, 1 / np.sqrt(d), causal)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_attention_longer_sequence(it, oracle):
    """src/ops/flash_attention.rs:302-330: batch 1, heads 2, seq 128, head_dim 32, causal."""
    b, h, s, d = 1, 2, 128, 32
    x = _sin_fill(b * h * s * d, 0.01, 0.3).reshape(b, h, s, d)
    out = it.flash_attention(_t(it, x), _t(it, x), _t(it, x), True).numpy()
    xs = _to_bshd(x)
    std = _to_bshd(it.attention(_t(it, xs), _t(it, xs), _t(it, xs), True).numpy())
    assert np.max(np.abs(out - std)) < 1e-3
    ref, _ = oracle.attention_fwd_bhsd(x, x, x, 1 / np.sqrt(d), True)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_attention_output_shape(it, oracle):
    """src/ops/flash_attention.rs:332-349: batch 2, heads 8, seq 64, head_dim 64 (the fused
    kernels), causal; the shape, and the values against the oracle."""
    b, h, s, d = 2, 8, 64, 64
    x = _sin_fill(b * h * s * d, 0.001, 1.0).reshape(b, h, s, d)
    out = it.flash_attention(_t(it, x), _t(it, x), _t(it, x), True)
    assert out.shape() == [b, h, s, d]
    ref, _ = oracle.attention_fwd_bhsd(x, x, x, 1 / np.sqrt(d), True)
    assert normwise_rel(out.numpy(), ref) <= FP32_TOL


@pytest.mark.parametrize("d", [8, 16, 48, 64, 96, 128])
@pytest.mark.parametrize("s,causal", [(37, True), (130, False), (130, True)])
def test_flash_attention_head_dims(it, oracle, d, s, causal):
    """Every head size up to the reference's limit: 64 through the fused kernels, the rest through
    the materialised contractions behind the same entry point."""
    print(f"[flash bhsd] d={d} s={s} causal={causal}", flush=True)
    b, h = 2, 3
    q, k, v = (synth.normal(300 + d + i, (b, h, s, d)) for i in range(3))
    out = it.flash_attention(_t(it, q), _t(it, k), _t(it, v), causal).numpy()
    ref, _ = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(d), causal)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_attention_tiny_shape(it, oracle):
    """The TINY layer's attention as the reference trainer calls it (src/train/forward.rs:124-138):
    [16, 4, 256, 64], causal, through the fused kernels."""
    b, h, s, d = 16, 4, 256, 64
    q, k, v = (synth.normal(320 + i, (b, h, s, d)) for i in range(3))
    out = it.flash_attention(_t(it, q), _t(it, k), _t(it, v), True).numpy()
    ref, _ = oracle.attention_fwd_bhsd(q, k, v, 1 / np.sqrt(d), True)
    assert normwise_rel(out, ref) <= FP32_TOL


def test_flash_attention_contract_errors(it):
    """The reference's assertions (src/ops/flash_attention.rs:77-98) and its zeros at seq 0."""
    x = _t(it, synth.normal(5, (1, 2, 8, 32)))
    with pytest.raises(it.Panic, match="Q must be FP32"):
        it.flash_attention(it.Tensor.from_f32_as_bf16(synth.normal(5, (1, 2, 8, 32)), [1, 2, 8, 32]), x, x, False)
    with pytest.raises(it.Panic, match="Q must be 4D"):
        it.flash_attention(_t(it, synth.normal(6, (2, 8, 32))), x, x, False)
    with pytest.raises(it.Panic, match="Q and K must have same shape"):
        it.flash_attention(x, _t(it, synth.normal(7, (1, 2, 9, 32))), x, False)
    with pytest.raises(it.Panic, match="Q and V must have same shape"):
        it.flash_attention(x, x, _t(it, synth.normal(8, (1, 1, 8, 32))), False)
    big = _t(it, synth.normal(9, (1, 1, 4, 129)))
    with pytest.raises(it.Panic, match="head_dim must be <= 128"):
        it.flash_attention(big, big, big, False)
    z = it.Tensor.zeros([2, 3, 0, 64])
    out = it.flash_attention(z, z, z, True)
    assert out.shape() == [2, 3, 0, 64]


@pytest.mark.parametrize("d", [16, 32, 128])
def test_flash_backward_other_head_dims(it, oracle, d):
    """flash_attention_backward at head sizes other than 64 (the materialised recompute behind the
    same entry point) against the oracle; O and lse apply to head_dim 64 only."""
    b, h, s = 2, 2, 100
    q, k, v, do = (synth.normal(340 + d + i, (b, h, s, d)) for i in range(4))
    tq, tk, tv, tdo = (_t(it, x) for x in (q, k, v, do))
    got = it.flash_attention_backward(tdo, tq, tk, tv, causal=True)
    ref = oracle.attention_bwd_bhsd(do, q, k, v, 1 / np.sqrt(d), True)
    for name, g, r in zip("QKV", got, ref):
        assert normwise_rel(g.numpy(), r) <= FP32_TOL, name
    fake = it.Tensor.zeros([b, h, s, d])
    with pytest.raises(it.TensorError, match="head_dim 64 only"):
        it.flash_attention_backward(tdo, tq, tk, tv, causal=True, o=fake, lse=it.Tensor.zeros([b * h, s]))


def test_flash_rejects_bad_scale(it):
    """The fused kernels need a finite scale > 0 (the BF16 forward scales each row's maximum)."""
    x = _t(it, synth.normal(11, (1, 1, 16, 64)))
    for sc in (0.0, -0.125, float("inf")):
        with pytest.raises(it.TensorError, match="scale must be finite"):
            it.flash_attention_forward_bhsd(x, x, x, causal=False, scale=sc)


# ---------------------------------------------------- BF16 fused kernels at their edges (flash2)

def _bf(it, x):
    return it.Tensor.from_f32_as_bf16(x, x.shape)


@pytest.mark.parametrize("s", [100, 130, 200, 257])
@pytest.mark.parametrize("causal", [True, False])
def test_flash_bf16_ragged(it, oracle, s, causal):
    """BF16 forward and backward at lengths that leave partial 64- and 128-row tiles, causal and not,
    against the f32 oracle on the unrounded inputs (relative Frobenius 1e-2)."""
    print(f"[flash bf16 ragged] s={s} causal={causal}", flush=True)
    b, h = 2, 3
    q, k, v, do = (synth.normal(400 + s + i, (b, h, s, D)) for i in range(4))
    tq, tk, tv, tdo = (_bf(it, x) for x in (q, k, v, do))
    o, lse = it.flash_attention_forward_bhsd(tq, tk, tv, causal=causal, scale=0.125)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 0.125, causal)
    assert frob_rel(o.numpy(), ro) <= BF16_FROB_TOL
    _, rl = _softmax_f64(q.reshape(b * h, s, D), k.reshape(b * h, s, D), 0.125, causal)
    assert np.max(np.abs(lse.numpy() - rl)) < 2e-2 * max(1.0, np.max(np.abs(rl)))
    grads = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, scale=0.125, o=o, lse=lse)
    recomputed = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, scale=0.125)
    refs = oracle.attention_bwd_bhsd(do, q, k, v, 0.125, causal)
    for name, g, rc, r in zip("QKV", grads, recomputed, refs):
        gg = g.numpy()
        assert frob_rel(gg, r) <= BF16_FROB_TOL, name
        assert np.array_equal(gg, rc.numpy()), name  # the recompute runs the same forward kernel


@pytest.mark.parametrize("sq,skv", [(70, 200), (300, 130), (129, 257)])
def test_flash_bf16_kv_length_differs(it, sq, skv):
    """BF16 forward with seq_q != seq_kv (non-causal), against float64 softmax on the f32 inputs."""
    b, h = 2, 2
    q = synth.normal(500 + sq, (b, h, sq, D))
    k = synth.normal(501 + skv, (b, h, skv, D))
    v = synth.normal(502 + skv, (b, h, skv, D))
    o, lse = it.flash_attention_forward_bhsd(_bf(it, q), _bf(it, k), _bf(it, v), causal=False, scale=0.125)
    p, rl = _softmax_f64(q.reshape(b * h, sq, D), k.reshape(b * h, skv, D), 0.125, False)
    ref = (p @ v.reshape(b * h, skv, D).astype(np.float64)).reshape(b, h, sq, D)
    assert frob_rel(o.numpy(), ref) <= BF16_FROB_TOL
    assert np.max(np.abs(lse.numpy() - rl)) < 2e-2 * max(1.0, np.max(np.abs(rl)))


def _raw_flash(it, prec, q, k, v, do, causal, lq, lkv, b, h, sq, skv):
    """Fused forward, then backward (when do is given), through the C ABI with explicit layouts."""
    import ctypes as C

    from irontensor_amd import _lib
    ctx = it.Context.global_()
    dt = _lib.IT_BF16 if prec == "bf16" else _lib.IT_F32
    vp = lambda t: C.c_void_p(t.ptr)  # noqa: E731
    o = it.Tensor.empty([b, sq, h, D])
    lse = it.Tensor.empty([b * h, sq])
    st = ctx.lib.it_flash_attention_forward(ctx.handle, dt, b * h, sq, skv, D, C.c_float(0.125), int(causal),
                                            C.byref(lq), C.byref(lkv), C.byref(lq), vp(q), vp(k), vp(v), vp(o),
                                            vp(lse))
    assert st == 0, _lib.last_error()
    if do is None:
        return o, None
    grads = [it.Tensor.empty([b, sq, h, D]) for _ in range(3)]
    st = ctx.lib.it_flash_attention_backward(ctx.handle, dt, b * h, sq, D, C.c_float(0.125), int(causal),
                                             C.byref(lq), C.byref(lkv), C.byref(lq), vp(do), vp(q), vp(k), vp(v),
                                             vp(o), vp(lse), *(vp(g) for g in grads))
    assert st == 0, _lib.last_error()
    return o, grads


@pytest.mark.parametrize("causal", [True, False])
def test_flash_bf16_bshd_strided(it, oracle, causal):
    """BF16 forward and backward reading Q, K, V, dO in place from [B, S, H, D] tensors (per-head
    strides, as the medium step reads its fused QKV buffer), against the oracle."""
    from irontensor_amd import _lib
    b, s, h = 2, 200, 3
    q, k, v, do = (synth.normal(520 + i, (b, s, h, D)) for i in range(4))
    lay = _lib.AttnLayout(h, s * h * D, D, h * D)
    o, grads = _raw_flash(it, "bf16", *(_bf(it, x) for x in (q, k, v, do)), causal, lay, lay, b, h, s, s)
    tb = lambda x: np.ascontiguousarray(x.transpose(0, 2, 1, 3))  # noqa: E731  [B,S,H,D] -> [B,H,S,D]
    ro, _ = oracle.attention_fwd_bhsd(tb(q), tb(k), tb(v), 0.125, causal)
    assert frob_rel(tb(o.numpy()), ro) <= BF16_FROB_TOL
    refs = oracle.attention_bwd_bhsd(tb(do), tb(q), tb(k), tb(v), 0.125, causal)
    for name, g, r in zip("QKV", grads, refs):
        assert frob_rel(tb(g.numpy()), r) <= BF16_FROB_TOL, name


# ----------------------------------------- BF16 outputs (it_flash_attention_forward_ex / backward_ex)

@pytest.mark.parametrize("s,causal", [(1024, True), (200, False)])
def test_flash_bf16_outputs(it, oracle, s, causal):
    """BF16 O and dQ, dK, dV: the forward's BF16 O is the round-to-nearest-even of its FP32 O bit for
    bit; the recomputing backward's BF16 gradients are those of its FP32 gradients bit for bit; the
    backward reading the BF16 O stays within the BF16 contract of the oracle."""
    from irontensor_amd import bf16_to_f32, f32_to_bf16
    b, h = 2, 4
    B16 = it.Precision.BF16
    q, k, v, do = (synth.normal(700 + s + i, (b, h, s, D)) for i in range(4))
    tq, tk, tv, tdo = (_bf(it, x) for x in (q, k, v, do))
    o32, lse32 = it.flash_attention_forward_bhsd(tq, tk, tv, causal=causal, scale=0.125)
    o16, lse16 = it.flash_attention_forward_bhsd(tq, tk, tv, causal=causal, scale=0.125, out_precision=B16)
    assert o16.precision() is B16
    assert np.array_equal(o16.as_bf16_slice(), f32_to_bf16(o32.numpy()).ravel())
    assert np.array_equal(lse16.numpy(), lse32.numpy())
    g32 = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, scale=0.125)
    g16 = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, scale=0.125, out_precision=B16)
    for name, x, y in zip("QKV", g32, g16):
        assert np.array_equal(y.as_bf16_slice(), f32_to_bf16(x.numpy()).ravel()), name
    chained = it.flash_attention_backward(tdo, tq, tk, tv, causal=causal, scale=0.125, o=o16, lse=lse16,
                                          out_precision=B16)
    ro, _ = oracle.attention_fwd_bhsd(q, k, v, 0.125, causal)
    assert frob_rel(bf16_to_f32(o16.as_bf16_slice()).reshape(ro.shape), ro) <= BF16_FROB_TOL
    refs = oracle.attention_bwd_bhsd(do, q, k, v, 0.125, causal)
    for name, g, r in zip("QKV", chained, refs):
        assert g.precision() is B16
        assert frob_rel(g.numpy(), r) <= BF16_FROB_TOL, name


def test_flash_bf16_output_refusals(it):
    """A BF16 output needs BF16 operands and head_dim 64."""
    x32 = _t(it, synth.normal(12, (1, 2, 64, 64)))
    with pytest.raises(it.TensorError, match="BF16 output needs BF16 operands"):
        it.flash_attention_forward_bhsd(x32, x32, x32, out_precision=it.Precision.BF16)
    x16 = _bf(it, synth.normal(13, (1, 2, 64, 32)))
    with pytest.raises(it.TensorError, match="head_dim 64"):
        it.flash_attention_backward(x16, x16, x16, x16, out_precision=it.Precision.BF16)
